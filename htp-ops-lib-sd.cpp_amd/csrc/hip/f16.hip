// Packed-F16 GEMM with fused epilogue (opcodes 1 and 16) on gfx950.
//
// Contract (reference src/dsp/ops/mat_mul.c:937-1049):
//   a = fp16(x) (RNE)                                       :114-148
//   acc = sum_k a*W, FP32 accumulation on v_mfma_f32_16x16x32_f16
//   v = (float)fp16(acc) -- the HMX readout is an fp16 tile  :724-778
//   mode 0: v + bias; 1: GELU(v + bias); 2: QuickGELU(v + bias);
//   mode 3: v + bias stored channel-major y[c][m], c < channels  :788-882
// The fp32->fp16 activation conversion is fused into the A-tile staging.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "hb_internal.h"
#include "qkv_post.h"

namespace {

constexpr int kFragBytes = 1024;  // 16 x 32 fp16 operand tile, lane-ordered
constexpr int kStageK = 64;       // k per LDS stage (two MFMA k-steps)

// ---------------------------------------------------------------------------
// Permuted reference layout -> MFMA tile image.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void f16_prepack(uint4 *__restrict__ packed, const uint16_t *__restrict__ perm,
                                                  int k, int n) {
  const size_t slots = (size_t)n * (size_t)k / 8u;
  const int kblocks = k / 32;
  for (size_t slot = (size_t)blockIdx.x * blockDim.x + threadIdx.x; slot < slots;
       slot += (size_t)gridDim.x * blockDim.x) {
    const size_t blk = slot / 64u;
    const int lane = (int)(slot % 64u);
    const int nb = (int)(blk / (size_t)kblocks), kb = (int)(blk % (size_t)kblocks);
    const int col = nb * 16 + lane % 16;
    const int k0 = kb * 32 + (lane / 16) * 8;
    uint32_t w[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int kk = k0 + 2 * g;  // even: (kk, kk+1) are adjacent in the permuted layout
      const size_t idx = ((size_t)(col / 32) * (size_t)kblocks + (size_t)(kk / 32)) * 1024u +
                         (size_t)((kk % 32) / 2) * 64u + (size_t)(col % 32) * 2u;
      w[g] = *(const uint32_t *)(perm + idx);
    }
    packed[slot] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---------------------------------------------------------------------------
// Dequantizing prepack (opcodes 2/3/4): Q4_0 / Q8_0 / IQ4_NL super-blocks of
// 256 weights -> the same MFMA tile image as f16_prepack, so the GEMM is the
// F16 one.  Super-block b holds positions [256b, 256b + 256) of the permuted
// F16 layout (reference src/dsp/ops/mat_mul.c:1700-1712).  Position j uses
// fp16 scale j/32.  Q8_0: quant byte j.  Q4_0 / IQ4_NL: the four 64-value
// vectors of a super-block come from the low nibbles of the even bytes, the
// low nibbles of the odd bytes, then the high nibbles of the even and of the
// odd bytes (vlut16 splits even and odd source bytes, :401-427); Q4_0 values
// are nibble - 8, IQ4_NL values ggml's code book (:30-37).  value * scale is
// exact in fp32 and rounded once to fp16.
// ---------------------------------------------------------------------------

__constant__ int8_t kIq4NlValues[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

__device__ inline uint16_t qk0_value(const uint8_t *__restrict__ blk, int j, int type) {
  const int g = j / 32;
  const uint16_t sbits = (uint16_t)(blk[2 * g] | (blk[2 * g + 1] << 8));
  const float scale = (float)__builtin_bit_cast(_Float16, sbits);
  int q;
  if (type == HB_GGML_Q8_0) {
    q = (int8_t)blk[16 + j];
  } else {
    const int v = j / 64, lane = j % 64;
    const uint8_t byte = blk[16 + 2 * lane + (v & 1)];
    const int nib = v < 2 ? (byte & 15) : (byte >> 4);
    q = type == HB_GGML_IQ4_NL ? (int)kIq4NlValues[nib] : nib - 8;
  }
  float v = __fmul_rn((float)q, scale);
  // Keeps the product and the conversion apart: fused, they become
  // v_fma_mix(q, scale, +0), which turns a -0 product (code 0, negative
  // scale) into +0.
  asm volatile("" : "+v"(v));
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

__global__ __launch_bounds__(256) void qk0_prepack(uint4 *__restrict__ packed, const uint8_t *__restrict__ blocks,
                                                  int k, int n, int type, int block_bytes) {
  const size_t slots = (size_t)n * (size_t)k / 8u;
  const int kblocks = k / 32;
  for (size_t slot = (size_t)blockIdx.x * blockDim.x + threadIdx.x; slot < slots;
       slot += (size_t)gridDim.x * blockDim.x) {
    const size_t blk = slot / 64u;
    const int lane = (int)(slot % 64u);
    const int nb = (int)(blk / (size_t)kblocks), kb = (int)(blk % (size_t)kblocks);
    const int col = nb * 16 + lane % 16;
    const int k0 = kb * 32 + (lane / 16) * 8;
    uint32_t w[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int kk = k0 + 2 * g;  // even: (kk, kk+1) are adjacent in the permuted layout
      const size_t idx = ((size_t)(col / 32) * (size_t)kblocks + (size_t)(kk / 32)) * 1024u +
                         (size_t)((kk % 32) / 2) * 64u + (size_t)(col % 32) * 2u;
      const uint8_t *sb = blocks + (idx / 256u) * (size_t)block_bytes;
      const int j = (int)(idx % 256u);
      w[g] = (uint32_t)qk0_value(sb, j, type) | ((uint32_t)qk0_value(sb, j + 1, type) << 16);
    }
    packed[slot] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---------------------------------------------------------------------------
// Epilogue activations (reference src/dsp/ops/mat_mul.c:788-826): stable
// sigmoid with e = 2^max(-|a|*log2(e), -126), by the hardware's v_exp_f32
// and v_rcp_f32 (each within 1 ulp; 1 + e lies in [1, 2]), far inside the
// F16 output bound.
// ---------------------------------------------------------------------------

__device__ inline float stable_sigmoid(float a) {
  const float neg = fmaxf(__fmul_rn(fabsf(a), -1.4426950408889634f), -126.0f);
  const float e = __builtin_amdgcn_exp2f(neg);
  const float inv = __builtin_amdgcn_rcpf(__fadd_rn(e, 1.0f));
  return a < 0.0f ? __fmul_rn(e, inv) : inv;
}

__device__ inline float apply_mode(float z, int mode) {
  if (mode == 1) {
    const float cubic = __fmul_rn(__fmul_rn(z, z), z);
    const float inner = __fadd_rn(z, __fmul_rn(cubic, 0.044715f));
    return __fmul_rn(z, stable_sigmoid(__fmul_rn(inner, 1.5957691216057308f)));
  }
  if (mode == 2) return __fmul_rn(z, stable_sigmoid(__fmul_rn(z, 1.702f)));
  return z;
}

// ---------------------------------------------------------------------------
// Tiled GEMM: BM x BN tile per workgroup of WM x WN waves; LDS double buffer
// of 64-k stages; A converted fp32 -> fp16 while staging.
// ---------------------------------------------------------------------------

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM *WN) void f16_gemm_tiles(float *__restrict__ y, const float *__restrict__ x,
                                                              const uint16_t *__restrict__ packed,
                                                              const float *__restrict__ bias, int m, int k, int n,
                                                              int channels, int mode) {
  constexpr int NT = 64 * WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int A_BYTES = BM * kStageK * 2, B_BYTES = BN * kStageK * 2;
  constexpr int A_CH = BM * 8 / NT;  // 8 fp16 (one 16-byte slot) per chunk
  constexpr int B_CH = B_BYTES / 16 / NT;
  static_assert(A_CH * NT == BM * 8 && B_CH * 16 * NT == B_BYTES, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][A_BYTES + B_BYTES];

  const int tiles_n = (n + BN - 1) / BN;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kblocks = k / 32;
  const int stages = (k + kStageK - 1) / kStageK;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;

  const float *a_src[A_CH];
  int a_dst[A_CH], a_k[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + NT * i;
    const int row = c >> 3, kc = c & 7;  // kc: 8-element chunk within the 64-k stage
    const int grow = min(m0 + row, m - 1);
    a_src[i] = x + (size_t)grow * k + kc * 8;
    a_k[i] = kc * 8;
    a_dst[i] = ((row >> 4) * 2 + (kc >> 2)) * kFragBytes + ((row & 15) + 16 * (kc & 3)) * 16;
  }
  const uint16_t *b_src[B_CH];
  int b_dst[B_CH], b_kb[B_CH];
  const int nblocks = n / 16;
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + NT * i;
    const int blk = c >> 7, rem = c & 127;
    const int kb2 = rem >> 6, slot = rem & 63;
    const int gnb = min(n0 / 16 + blk, nblocks - 1);
    b_src[i] = packed + ((size_t)gnb * kblocks + kb2) * 512u + slot * 8;
    b_kb[i] = kb2;
    b_dst[i] = A_BYTES + (blk * 2 + kb2) * kFragBytes + slot * 16;
  }

  uint4 ra[A_CH], rb[B_CH];
  auto load = [&](int st) {
    const int kbase = st * kStageK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      if (kbase + a_k[i] < k) {
        const float4 lo = *(const float4 *)(a_src[i] + kbase);
        const float4 hi = *(const float4 *)(a_src[i] + kbase + 4);
        hb_f16x8 h = {(_Float16)lo.x, (_Float16)lo.y, (_Float16)lo.z, (_Float16)lo.w,
                      (_Float16)hi.x, (_Float16)hi.y, (_Float16)hi.z, (_Float16)hi.w};
        ra[i] = *(const uint4 *)&h;
      } else {
        ra[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int kb = st * 2 + b_kb[i];
      rb[i] = kb < kblocks ? *(const uint4 *)(b_src[i] + (size_t)st * 2u * 512u) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *(uint4 *)(&lds[buf][a_dst[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *(uint4 *)(&lds[buf][b_dst[i]]) = rb[i];
  };

  hb_f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  load(0);
  stash(0);
  __syncthreads();
  for (int st = 0; st < stages; ++st) {
    const int cur = st & 1;
    if (st + 1 < stages) load(st + 1);
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      hb_f16x8 bf[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *(const hb_f16x8 *)(&lds[cur][A_BYTES + ((wn * FN + j) * 2 + kb2) * kFragBytes + lane * 16]);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const hb_f16x8 af = *(const hb_f16x8 *)(&lds[cur][((wm * FM + i) * 2 + kb2) * kFragBytes + lane * 16]);
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    if (st + 1 < stages) stash(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = n0 + wn * WTN + j * 16 + (lane & 15);
    const int limit = mode == 3 ? channels : n;
    if (col >= limit) continue;
    const float b = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
        if (row >= m) continue;
        const float v = (float)(_Float16)acc[i][j][r];
        const float z = bias ? __fadd_rn(v, b) : v;
        if (mode == 3) {
          y[(size_t)col * m + row] = z;
        } else {
          y[(size_t)row * n + col] = apply_mode(z, mode);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large M: both operands as 1 KB fp16 tiles in MFMA lane order, streamed
// through the direct-to-LDS ring of the int8 GEMM.  f16_pack_a converts the
// activations once per call (fp32 -> fp16 RNE, 16 rows x 32 k per tile, rows
// past m zero); the packed weights already have this form.  The k loop is the
// same sequence of v_mfma_f32_16x16x32_f16 per accumulator as f16_gemm_tiles,
// so the results are identical to it.
// ---------------------------------------------------------------------------

#include "hb_lds_ring.h"
static_assert(kFragBytes == kRingTileBytes, "operand tiles are the ring's tiles");

__global__ __launch_bounds__(256) void f16_pack_a(uint4 *__restrict__ img, const float *__restrict__ x, int m, int k,
                                                 int mp) {
  const size_t slots = (size_t)mp * (size_t)k / 8u;
  const int kblocks = k / 32;
  for (size_t slot = (size_t)blockIdx.x * blockDim.x + threadIdx.x; slot < slots;
       slot += (size_t)gridDim.x * blockDim.x) {
    const size_t tile = slot / 64u;
    const int lane = (int)(slot % 64u);
    const int mb = (int)(tile / (size_t)kblocks), kb = (int)(tile % (size_t)kblocks);
    const int row = mb * 16 + (lane & 15);
    const int k0 = kb * 32 + 8 * (lane >> 4);
    uint4 out = make_uint4(0u, 0u, 0u, 0u);
    if (row < m) {
      const float *xr = x + (size_t)row * k + k0;
      const hb_f32x4 lo = __builtin_nontemporal_load((const hb_f32x4 *)xr);
      const hb_f32x4 hi = __builtin_nontemporal_load((const hb_f32x4 *)(xr + 4));
      const hb_f16x8 h = {(_Float16)lo[0], (_Float16)lo[1], (_Float16)lo[2], (_Float16)lo[3],
                          (_Float16)hi[0], (_Float16)hi[1], (_Float16)hi[2], (_Float16)hi[3]};
      out = __builtin_bit_cast(uint4, h);
    }
    img[slot] = out;
  }
}

// ---------------------------------------------------------------------------
// Many rows, few columns (VAE convolutions as im2col GEMMs: M pixels,
// K = channels x 9, N output channels): the fp32 activations are the bulk of
// the bytes, so they stream from HBM once, straight into registers (lane l
// loads 8 values of row l % 16 per k-step as two float4, converted to fp16
// there: the MFMA operand layout), while each k-step's weight fragments of
// the workgroup's BN columns pass through an LDS ring that its waves fill
// together (global_load_lds).  Each wave owns 16 rows x BN columns; the
// loads of k-step kt + D are issued while k-step kt multiplies, unconditional
// (past the end they repeat the last k-step, unused), so every wait counts
// exactly D - 1 later k-steps of loads.  A workgroup covers BN columns;
// larger n takes several column chunks, those of one row block dispatched
// together so that the activation re-reads find the memory-side cache.
// SWAP (row-major output, modes 0-2): the weights are the MFMA A operand, so
// a lane holds 4 consecutive columns of one row and stores them as one
// 16-byte vector; mode 3 (channel-major [channels][m]) keeps the activations
// as the A operand, so a lane holds 4 consecutive rows of one channel.  The
// k-steps are multiplied in order, one v_mfma_f32_16x16x32_f16 per 32 k, as
// in f16_gemm_tiles, so the sums are the same.  Requires k % 32 == 0,
// n % 16 == 0, 16-byte aligned x (and y for SWAP).
// ---------------------------------------------------------------------------
// k-step kt's weights into its ring stage (instruction i of the wave fills
// fragment i * WAVES + wave); past the last k-step the last one is read
// again (never used).
template <int PW, int WAVES, int S, int STAGE>
__device__ __attribute__((always_inline)) inline void xstream_issue_w(int8_t *lds, const int8_t *const *bsrc, int kt,
                                                                     int kt_count, int wave) {
  const int kc = min(kt, kt_count - 1);
  int8_t *stage = lds + (kt % S) * STAGE;
#pragma unroll
  for (int i = 0; i < PW; ++i)
    __builtin_amdgcn_global_load_lds(bsrc[i] + (size_t)kc * kFragBytes,
                                     HB_LDS_PTR(stage + (i * WAVES + wave) * kFragBytes), 16, 0, 0);
}

// A wave's 16 rows x 32 activations of one k-step: two DMA instructions, each
// bringing 8 whole 128-byte rows (16-byte piece p of row r' by the lane in
// slot (8p + r') ^ 8i), into a 2 KB slot of the wave's own LDS queue.
__device__ __attribute__((always_inline)) inline void xstream_issue_a(int8_t *slot, const float *const *arow, int kt,
                                                                     int kt_count) {
  const int kc = min(kt, kt_count - 1);
#pragma unroll
  for (int i = 0; i < 2; ++i)
    __builtin_amdgcn_global_load_lds(arow[i] + 32 * kc, HB_LDS_PTR(slot + i * 1024), 16, 0, 0);
}

// DA: k-steps of activations in flight (a queue of DA 2 KB slots per wave in
// LDS), DB: k-steps of weights in flight (a ring of DB + 1 stages shared by
// the waves): the activations come from HBM and need the deeper queue, the
// weights (a few MB read by every workgroup) mostly hit L2.
template <int BN, int WAVES, int DA, int DB, bool SWAP>
__global__ __launch_bounds__(64 * WAVES) void f16_gemm_xstream(float *__restrict__ y, const float *__restrict__ x,
                                                              const int8_t *__restrict__ wpack,
                                                              const float *__restrict__ bias, int m, int k, int n,
                                                              int channels, int mode) {
  constexpr int FN = BN / 16;                 // column fragments
  constexpr int S = DB + 1;                   // weight ring stages
  constexpr int STAGE = FN * kFragBytes;      // one k-step of the chunk's weights
  constexpr int PW = FN / WAVES;              // weight DMA instructions per wave and k-step
  constexpr int ASLOT = 2048;                 // one k-step of a wave's activations
  // k-step kt waits for its weights (issued at step kt - DB, before that
  // step's activation DMA) and its activations (issued at kt - DA <= kt - DB):
  // younger are the whole groups of the DB - 1 steps after kt - DB, and the 2
  // activation DMA of step kt - DB itself when they are a later k-step's
  // (DA > DB; with DA == DB they are k-step kt's own)
  constexpr int LATER = (DA > DB ? 2 : 0) + (DB - 1) * (PW + 2);
  static_assert(PW * WAVES == FN && PW >= 1, "every wave issues the same weight DMA count");
  static_assert(FN % 4 == 0, "fragments are read four at a time");
  static_assert(DA >= DB && DB >= 1, "activations at least as far ahead as weights");
  static_assert(LATER < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE + WAVES * DA * ASLOT];

  // Workgroups are dealt to the 8 XCDs in turn (bid % 8).  With several
  // column chunks and whole groups of 8 row blocks, the chunks of one row
  // block are bid, bid + 8, ...: the same XCD, dispatched together, so the
  // later chunks read the rows from that XCD's L2.
  const int chunks = (n + BN - 1) / BN, tiles_m = (m + 16 * WAVES - 1) / (16 * WAVES);
  const int bid = blockIdx.x;
  int tm, tn;
  if (chunks > 1 && tiles_m % 8 == 0) {
    tm = (bid / (8 * chunks)) * 8 + bid % 8;
    tn = (bid / 8) % chunks;
  } else {
    tm = bid / chunks;
    tn = bid % chunks;
  }
  const int m0 = tm * 16 * WAVES, n0 = tn * BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kt_count = k / 32, nblocks = n / 16;

  const int8_t *bsrc[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int nb = min(n0 / 16 + i * WAVES + wave, nblocks - 1);
    bsrc[i] = wpack + (size_t)nb * kt_count * kFragBytes + lane * 16;
  }
  // this lane's activation piece in DMA instruction i: row 8i + r', piece p
  const float *arow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int v = lane ^ (8 * i), p = v >> 3, r = v & 7;
    arow[i] = x + (size_t)min(m0 + wave * 16 + 8 * i + r, m - 1) * k + 4 * p;
  }
  int8_t *const aq = lds + S * STAGE + wave * DA * ASLOT;  // this wave's activation queue
  const uint32_t lds_addr = (uint32_t)(uintptr_t)HB_LDS_PTR(lds);
  const uint32_t aq_addr = (uint32_t)(uintptr_t)HB_LDS_PTR(aq);
  // where lane l (row l % 16, values 8 (l / 16) .. + 7) finds its two pieces
  const int ar = lane & 15, aq2 = 2 * (lane >> 4);
  const uint32_t a_lo = (uint32_t)((ar >> 3) * 64 + ((8 * aq2 + (ar & 7)) ^ (8 * (ar >> 3)))) * 16u;
  const uint32_t a_hi = (uint32_t)((ar >> 3) * 64 + ((8 * (aq2 + 1) + (ar & 7)) ^ (8 * (ar >> 3)))) * 16u;
  hb_f32x4 acc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) acc[j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // the groups of steps -DA .. -1, as the main loop would have issued them
#pragma unroll
  for (int s = -DA; s < 0; ++s) {
    if (s + DB >= 0) xstream_issue_w<PW, WAVES, S, STAGE>(lds, bsrc, s + DB, kt_count, wave);
    xstream_issue_a(aq + ((s + DA) % DA) * ASLOT, arow, s + DA, kt_count);
  }
  // One k-step.  After the wait this wave's DMA of k-step kt have landed;
  // after the barrier every wave's have, and every wave is done with the
  // weight stage k-step kt + DB reuses.  The activations are read (and their
  // slot refilled with k-step kt + DA) first, then the weight fragments.
  // All LDS reads are instructions the compiler does not track: it cannot
  // tell the bytes read from the DMA targets in flight and would wait for
  // every one of them (vmcnt(0)) before each read; the wait and the barrier
  // cover the bytes read.
#define XSTREAM_STEP(KT)                                                                                           \
  do {                                                                                                             \
    const int kt_ = (KT);                                                                                          \
    wait_vmcnt<LATER>();                                                                                           \
    block_barrier();                                                                                               \
    const uint32_t aslot = aq_addr + (uint32_t)((kt_ % DA) * ASLOT);                                               \
    hb_f32x4 lo, hi;                                                                                               \
    asm volatile("ds_read_b128 %0, %1" : "=v"(lo) : "v"(aslot + a_lo));                                            \
    asm volatile("ds_read_b128 %0, %1" : "=v"(hi) : "v"(aslot + a_hi));                                            \
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo), "+v"(hi));                                                     \
    const hb_f16x8 af = {(_Float16)lo[0], (_Float16)lo[1], (_Float16)lo[2], (_Float16)lo[3],                      \
                         (_Float16)hi[0], (_Float16)hi[1], (_Float16)hi[2], (_Float16)hi[3]};                      \
    xstream_issue_w<PW, WAVES, S, STAGE>(lds, bsrc, kt_ + DB, kt_count, wave);                                    \
    xstream_issue_a(aq + (kt_ % DA) * ASLOT, arow, kt_ + DA, kt_count);                                            \
    const uint32_t base = lds_addr + (uint32_t)((kt_ % S) * STAGE + lane * 16);                                   \
    _Pragma("unroll") for (int j0 = 0; j0 < FN; j0 += 4) {                                                        \
      hb_u32x4 f[4];                                                                                               \
      _Pragma("unroll") for (int q = 0; q < 4; ++q) asm volatile("ds_read_b128 %0, %1"                            \
                                                                 : "=v"(f[q])                                     \
                                                                 : "v"(base + (uint32_t)((j0 + q) * kFragBytes)));  \
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));                     \
      _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                                             \
        const hb_f16x8 bf = __builtin_bit_cast(hb_f16x8, f[q]);                                                    \
        acc[j0 + q] = SWAP ? __builtin_amdgcn_mfma_f32_16x16x32_f16(bf, af, acc[j0 + q], 0, 0, 0)                 \
                           : __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[j0 + q], 0, 0, 0);                \
      }                                                                                                            \
    }                                                                                                              \
  } while (0)
  for (int kt = 0; kt < kt_count; ++kt) XSTREAM_STEP(kt);
#undef XSTREAM_STEP
  wait_vmcnt<0>();  // no weight DMA may still write this workgroup's LDS when it ends

  if constexpr (SWAP) {
    // lane l: row m0 + 16 wave + l % 16, columns n0 + 16 j + 4 (l / 16) .. + 3
    const int row = m0 + wave * 16 + (lane & 15);
    if (row >= m) return;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + j * 16 + 4 * (lane >> 4);
      if (col >= n) continue;
      float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (bias) {
#pragma unroll
        for (int r = 0; r < 4; ++r) b[r] = bias[col + r];
      }
      hb_f32x4 out;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (float)(_Float16)acc[j][r];
        out[r] = apply_mode(bias ? __fadd_rn(v, b[r]) : v, mode);
      }
      __builtin_nontemporal_store(out, (hb_f32x4 *)(y + (size_t)row * n + col));
    }
  } else {
    // lane l: rows m0 + 16 wave + 4 (l / 16) .. + 3, column n0 + 16 j + l % 16
    const int row0 = m0 + wave * 16 + 4 * (lane >> 4);
    const bool whole = row0 + 3 < m && (m & 3) == 0;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + j * 16 + (lane & 15);
      if (col >= channels) continue;
      const float b = bias ? bias[col] : 0.0f;
      hb_f32x4 out;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (float)(_Float16)acc[j][r];
        out[r] = bias ? __fadd_rn(v, b) : v;
      }
      float *dst = y + (size_t)col * m + row0;
      if (whole) {
        __builtin_nontemporal_store(out, (hb_f32x4 *)dst);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (row0 + r < m) dst[r] = out[r];
      }
    }
  }
}

// The k loop of the ring kernels: tile (m0, n0) of the product into acc (the
// MFMA layout: lane l holds rows 4*(l/16)..+3 and column l%16 of each 16x16
// block of this wave's WTM x WTN sub-tile).  On return every operand stage
// has been consumed, so the caller may reuse the LDS after a barrier.
template <int BM, int BN, int WM, int WN, int S>
__device__ inline void ring_mainloop(hb_f32x4 (&acc)[BM / WM / 16][BN / WN / 16], int8_t *lds,
                                     const int8_t *__restrict__ aimg, const int8_t *__restrict__ wpack, int m, int k,
                                     int n, int m0, int n0, int wave, int lane, int kt0 = 0, int kt_n = -1) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int ABLK = BM / 16, BBLK = BN / 16;
  constexpr int NB = ABLK + BBLK;
  constexpr int PW = (NB + NW - 1) / NW;
  constexpr int PW_LO = NB / NW;
  static_assert(PW_LO >= 1, "every wave takes part in the DMA");
  constexpr int STAGE = NB * kFragBytes;
  const int kt_count = k / 32;  // k-steps of a whole row (the operand block stride)
  const int wm = wave / WN, wn = wave % WN;
  // k-steps [kt0, kt0 + steps) of the product (all of them by default)
  const int steps = kt_n < 0 ? kt_count : kt_n;

  const int8_t *src[PW];
  int stride[PW];
  const int nblocks = n / 16;
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int b = min(i * NW + wave, NB - 1);
    if (b < ABLK) {
      const int mb = min(m0 / 16 + b, (m + 15) / 16 - 1);
      src[i] = aimg + (size_t)mb * kt_count * kFragBytes + lane * 16;
    } else {
      const int nb = min(n0 / 16 + (b - ABLK), nblocks - 1);
      src[i] = wpack + (size_t)nb * kt_count * kFragBytes + lane * 16;
    }
    stride[i] = kFragBytes;
  }

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < steps) dma_stage<PW, NW, NB>(lds + (s % S) * STAGE, src, stride, kt0 + s, wave, lane);
  for (int kt = 0; kt < steps; ++kt) {
    if (PW == PW_LO || wave < NB % NW)
      wait_stage<PW, S - 2>(steps - 1 - kt);
    else
      wait_stage<PW_LO, S - 2>(steps - 1 - kt);
    block_barrier();
    if (kt + S - 1 < steps)
      dma_stage<PW, NW, NB>(lds + ((kt + S - 1) % S) * STAGE, src, stride, kt0 + kt + S - 1, wave, lane);
    const int8_t *base = lds + (kt % S) * STAGE;
    const int8_t *la = base + (wm * FM) * kFragBytes + lane * 16;
    const int8_t *lb = base + (ABLK + wn * FN) * kFragBytes + lane * 16;
    hb_f16x8 bf[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const hb_f16x8 *)(lb + j * kFragBytes);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const hb_f16x8 af = *(const hb_f16x8 *)(la + i * kFragBytes);
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
    }
  }
}

template <int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * WM *WN) void f16_gemm_ring(float *__restrict__ y, const int8_t *__restrict__ aimg,
                                                             const int8_t *__restrict__ wpack,
                                                             const float *__restrict__ bias, int m, int k, int n,
                                                             int channels, int mode) {
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int STAGE = (BM / 16 + BN / 16) * kFragBytes;
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE];

  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
  int tm, tn;
  tile_coords_2d<BM, BN>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  hb_f32x4 acc[FM][FN];
  ring_mainloop<BM, BN, WM, WN, S>(acc, lds, aimg, wpack, m, k, n, m0, n0, wave, lane);

  const int row0 = m0 + wm * WTM;
  const int col0 = n0 + wn * WTN;
  if (mode == 3) {
    // Channel-major output y[channels][m] (columns past channels dropped):
    // lane l holds rows 4*(l/16)..+3 of column l%16 of each 16x16 block, one
    // 16-byte store along M (element stores when m is not a multiple of 4).
    const bool vec = (m & 3) == 0;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = col0 + j * 16 + (lane & 15);
      if (col >= channels) continue;
      const float b = bias ? bias[col] : 0.0f;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r0 = row0 + i * 16 + 4 * (lane >> 4);
        if (r0 >= m) continue;
        hb_f32x4 out;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = (float)(_Float16)acc[i][j][r];
          out[r] = bias ? __fadd_rn(v, b) : v;
        }
        float *dst = y + (size_t)col * m + r0;
        if (vec) {
          __builtin_nontemporal_store(out, (hb_f32x4 *)dst);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r0 + r < m) dst[r] = out[r];
        }
      }
    }
    return;
  }

  // Epilogue: fp16 readout, bias, activation, then each 16-row chunk staged
  // in wave-private padded LDS and written as 16-byte vectors along rows.
  float bj[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) bj[j] = bias ? bias[min(col0 + j * 16 + (lane & 15), n - 1)] : 0.0f;
  block_barrier();  // every wave is done with the operand stages: LDS becomes staging
  constexpr int SROW = WTN + 4;
  static_assert(16 * SROW * 4 * NW <= S * STAGE, "staging must fit in the operand LDS");
  float *stg = (float *)lds + wave * 16 * SROW;
  constexpr int VPR = WTN / 4;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (float)(_Float16)acc[i][j][r];
        const float z = bias ? __fadd_rn(v, bj[j]) : v;
        stg[((lane >> 4) * 4 + r) * SROW + j * 16 + (lane & 15)] = apply_mode(z, mode);
      }
#pragma unroll
    for (int v = lane; v < 16 * VPR; v += 64) {
      const int r = v / VPR, c4 = v % VPR;
      const int row = row0 + i * 16 + r, col = col0 + c4 * 4;
      if (row < m && col < n) {
        const hb_f32x4 val = *(const hb_f32x4 *)(stg + r * SROW + c4 * 4);
        __builtin_nontemporal_store(val, (hb_f32x4 *)(y + (size_t)row * n + col));
      }
    }
  }
}

// Split-K form of the ring kernel for up to 128 rows: grid (tiles, splits),
// split s multiplies k-steps [s*kps, s*kps + kps) of its BM x BN tile (the
// k loop of f16_gemm_ring on that range) and stores the raw fp32 sums to
// slice s of the workspace ([mp][n] per slice, rows past m dropped by the
// buffer bound); f16_skinny_epilogue then adds the slices in order, reads
// out to fp16 and applies bias and activation.  A tile covers every row, so
// the fp16 weights are read once, and the splits give the launch enough
// workgroups.
template <int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * WM *WN) void f16_ring_splitk(float *__restrict__ ws, const int8_t *__restrict__ aimg,
                                                               const int8_t *__restrict__ wpack, int m, int k, int n,
                                                               int kps, int channel_major) {
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int STAGE = (BM / 16 + BN / 16) * kFragBytes;
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE];
  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
  int tm, tn;
  tile_coords_2d<BM, BN>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  const int kt0 = blockIdx.y * kps, kt_n = min(kps, k / 32 - kt0);
  hb_f32x4 acc[FM][FN];
  ring_mainloop<BM, BN, WM, WN, S>(acc, lds, aimg, wpack, m, k, n, m0, n0, wave, lane, kt0, kt_n);
  // lane l holds rows 4*(l/16)..+3 and column l%16 of each 16x16 block
  const int mp = (m + 15) / 16 * 16;
  if (channel_major) {
    // slice s as [n][mp]: the lane's 4 rows of a column are one 16-byte store
    float *slice = ws + (size_t)blockIdx.y * mp * n;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * WTN + j * 16 + (lane & 15);
        const int r0 = m0 + wm * WTM + i * 16 + 4 * (lane >> 4);
        if (col < n && r0 < mp) *(hb_f32x4 *)(slice + (size_t)col * mp + r0) = acc[i][j];
      }
    return;
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(ws + (size_t)blockIdx.y * mp * n, 0, (uint32_t)m * (uint32_t)n * 4u, 0x00020000);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * WTN + j * 16 + (lane & 15);
      if (col >= n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * WTM + i * 16 + 4 * (lane >> 4) + r;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), rs, (uint32_t)(row * n + col) * 4u, 0, 0);
      }
    }
}

// ---------------------------------------------------------------------------
// Streaming F16 GEMM (persistent): the plan of the int8 streaming GEMM with
// fp16 operands.  One workgroup per CU walks its share of BM x BN tiles with
// one continuous operand ring, so the next tile's first k-steps are in flight
// while a tile finishes.
//  - ND DMA waves issue every operand DMA (buffer loads into LDS, 1 KB
//    lane-ordered blocks of the f16_pack_a image and of the packed weights)
//    and the tile's bias, wait for their own DMA only and publish each stage
//    with the workgroup barrier.  A wave's loads and stores complete in issue
//    order for its s_waitcnt count, so only waves that never store can wait
//    for one stage while output stores are still draining.
//  - WM x WN compute waves never load from global memory: each step they read
//    the next step's fragments from LDS while the current step's MFMAs run.
//    The weights are the MFMA's first operand, so a lane holds 4 consecutive
//    columns of one output row; every output element sees the k-steps in the
//    order f16_gemm_ring uses, so the bits are the same.  At a tile's end they
//    read out in registers (fp16 readout, bias, activation), trade halves of
//    each 16-lane row by DPP so that every store fills whole 128-byte lines,
//    and store without waiting: the stores drain during the next tile.
//  - The bias of a tile arrives in LDS with the tile's first stage, double
//    buffered by tile parity.
//  - The XCD that runs a workgroup (blockIdx % 8) owns a contiguous chunk of
//    the tiles in 4-row-block groups, so the blocks its workgroups share stay
//    in its L2.  Workgroups of odd slot start `stagger` ticks of the 100 MHz
//    real-time counter late, so that the two halves' tile ends, and the store
//    bursts after them, alternate.
// Requires gridDim.x % 8 == 0, k / 32 >= S - 1 (a tile's bias buffer is
// rewritten only after the tile two before it has finished), n % 32 == 0,
// and both operand images below 4 GB (32-bit buffer offsets).
// ---------------------------------------------------------------------------

// TAG (the kernel's activation mode) gives each kernel instantiation its own
// type: hipcc's host pass drops the launch stub of a kernel that shares this
// device-only type with another instantiation.
template <int BM, int BN, int ND, int TAG>
struct F16StreamDma {
  static constexpr int ABLK = BM / 16, NB = ABLK + BN / 16, PW = NB / ND;
  static_assert(NB % ND == 0 && ABLK % ND == 0 && BN * 4 <= kFragBytes, "DMA split");
  uint32_t soff[PW];    // byte offset of each block's k-step 0 in its operand image (uniform)
  const float *pbias;   // this lane's 16 bytes of the tile's bias (null: no bias)
  int tile, kt, slot;

  __device__ void point(int tm, int tn, const float *bias, int m, int n, int ktc, int d, int lane) {
    const int mblocks = (m + 15) / 16, nblocks = n / 16;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int b = i * ND + d;
      const int blk = i < ABLK / ND ? min(tm * ABLK + b, mblocks - 1) : min(tn * (BN / 16) + (b - ABLK), nblocks - 1);
      soff[i] = (uint32_t)blk * (uint32_t)ktc * (uint32_t)kFragBytes;
    }
    pbias = bias ? bias + min(tn * BN + 4 * min(lane, BN / 4 - 1), n - 4) : nullptr;
  }

  __device__ void issue(int8_t *lds, int stage_bytes, int8_t *params, int ktc, int S, int d, __amdgpu_buffer_rsrc_t ra,
                        __amdgpu_buffer_rsrc_t rb, uint32_t l16) {
    int8_t *dst = lds + slot * stage_bytes;
#pragma unroll
    for (int i = 0; i < PW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(i < ABLK / ND ? ra : rb, HB_LDS_PTR(dst + (i * ND + d) * kFragBytes), 16,
                                               l16, soff[i] + (uint32_t)kt * (uint32_t)kFragBytes, 0, 0);
    if (kt == 0 && d == 0 && pbias)
      __builtin_amdgcn_global_load_lds(pbias, HB_LDS_PTR(params + (tile & 1) * kFragBytes), 16, 0, 0);
    if (++kt == ktc) kt = 0;
    if (++slot == S) slot = 0;
  }
};

// One output element: fp16 readout of the fp32 sum, bias, activation.
template <int MODE>
__device__ inline uint32_t f16_out_bits(float acc, float b, bool has_bias) {
  const float v = (float)(_Float16)acc;
  const float z = has_bias ? __fadd_rn(v, b) : v;
  return __float_as_uint(apply_mode(z, MODE));
}

// DPP row shifts (within 16-lane rows): lane i takes lane i - 8 / lane i + 8.
constexpr int kDppRowShr8 = 0x118, kDppRowShl8 = 0x108;

template <int BM, int BN, int WM, int WN, int ND, int S, int MODE>
__global__ __launch_bounds__(64 * (WM * WN + ND), 1) void f16_gemm_stream(float *__restrict__ y,
                                                                         const int8_t *__restrict__ aimg,
                                                                         const int8_t *__restrict__ wpack,
                                                                         const float *__restrict__ bias, int m, int k,
                                                                         int n, int tiles_m, int tiles_n, int stagger) {
  constexpr int NW = WM * WN;  // compute waves 0..NW-1; DMA waves NW..NW+ND-1
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int ABLK = BM / 16;
  constexpr int STAGE = (ABLK + BN / 16) * kFragBytes;
  constexpr int SPLIT = FM < 2 ? FM : 2;  // row blocks of a step multiplied before the step's barrier
  static_assert(FN % 2 == 0, "column blocks in pairs (32 columns, one 128-byte line)");
  using Dma = F16StreamDma<BM, BN, ND, MODE>;
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE + 2 * kFragBytes];
  int8_t *params = lds + S * STAGE;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int ktc = k / 32;

  // This workgroup's tiles: chunk [c0, c1) of the grouped order belongs to its XCD.
  const int total = tiles_m * tiles_n;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8, nslots = gridDim.x / 8;
  const int per = (total + 7) / 8;
  const int c0 = min(total, xcd * per), c1 = min(total, c0 + per);
  const int ntile = c0 + slot < c1 ? (c1 - c0 - slot + nslots - 1) / nslots : 0;
  if (ntile == 0) return;
  const int steps = ntile * ktc;
  if (stagger > 0 && (slot & 1)) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < (uint64_t)stagger) __builtin_amdgcn_s_sleep(8);
  }

  if (wave >= NW) {
    // --------------------------------- DMA wave ---------------------------------
    // Stage g + 1 has landed once at most (S - 3) * PW of this wave's DMA
    // instructions are outstanding while the S - 3 stages after it have been
    // issued (a tile's first stage may carry the bias load besides, which only
    // makes the wait longer).  With fewer stages left: vmcnt(0).
    const int d = wave - NW;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)aimg, 0, (uint32_t)((m + 15) / 16) * (uint32_t)k * 32u, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)wpack, 0, (uint32_t)n * (uint32_t)k * 2u, 0x00020000);
    Dma dma;
    dma.tile = -1;
    dma.kt = 0;
    dma.slot = 0;
    auto next = [&]() {
      if (dma.kt == 0) {
        int tm, tn;
        group_tile(c0 + slot + (++dma.tile) * nslots, tiles_m, tiles_n, tm, tn);
        dma.point(tm, tn, bias, m, n, ktc, d, lane);
      }
      dma.issue(lds, STAGE, params, ktc, S, d, ra, rb, (uint32_t)lane * 16u);
    };
    static_assert(S >= 4, "at least one stage in flight behind the awaited one");
    for (int st = 0; st < S - 1 && st < steps; ++st) next();
    if (S - 1 <= steps) wait_vmcnt<(S - 2) * Dma::PW>(); else wait_vmcnt<0>();
    block_barrier();  // stage 0 published
    for (int g = 0; g < steps; ++g) {
      if (g + S - 2 < steps) wait_vmcnt<(S - 3) * Dma::PW>();
      else if (g + 1 < steps) wait_vmcnt<0>();
      block_barrier();  // stage g + 1 published; every compute wave is done with stage g - 1
      if (g + S - 1 < steps) next();  // into the slot stage g - 1 held
    }
    return;
  }

  // ------------------------------- compute wave -------------------------------
  const int wm = wave / WN, wn = wave % WN;
  hb_f32x4 acc[FM][FN];
  hb_f16x8 fa[2][FM], fb[2][FN];
  const int aoff = (wm * FM) * kFragBytes + lane * 16, boff = (ABLK + wn * FN) * kFragBytes + lane * 16;
  const int lcol = wn * WTN + 4 * (lane >> 4);                // tile column of this lane in block 0
  const int scol = 16 * ((lane >> 3) & 1) + 4 * (lane >> 4);  // column in a 32-column pair after the DPP trade
  const bool has_bias = bias != nullptr;
  block_barrier();  // stage 0 published
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < FM; ++i) fa[0][i] = *(const hb_f16x8 *)(lds + aoff + i * kFragBytes);
#pragma unroll
  for (int j = 0; j < FN; ++j) fb[0][j] = *(const hb_f16x8 *)(lds + boff + j * kFragBytes);
  int r = 0, kt = 0, rd_slot = 1 % S;  // tile and k-step of the step; slot of the next fragments

#define F16_STREAM_MFMA(P, I0, I1)                                                                          \
  _Pragma("unroll") for (int i = (I0); i < (I1); ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = \
      __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[P][j], fa[P][i], acc[i][j], 0, 0, 0);
#define F16_STREAM_STEP(P)                                                                                  \
  {                                                                                                         \
    F16_STREAM_MFMA(P, 0, SPLIT)                                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                                      \
    block_barrier();                                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                      \
    {                                                                                                       \
      /* unconditional (after the last step it reads a stale slot, unused): a branch here */                \
      /* would make the compiler wait for these reads before the MFMAs below */                             \
      const int8_t *base = lds + rd_slot * STAGE;                                                           \
      if (++rd_slot == S) rd_slot = 0;                                                                      \
      _Pragma("unroll") for (int i = 0; i < FM; ++i) fa[1 - (P)][i] =                                       \
          *(const hb_f16x8 *)(base + aoff + i * kFragBytes);                                                \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) fb[1 - (P)][j] =                                       \
          *(const hb_f16x8 *)(base + boff + j * kFragBytes);                                                \
    }                                                                                                       \
    __builtin_amdgcn_sched_barrier(0);                                                                      \
    F16_STREAM_MFMA(P, SPLIT, FM)                                                                           \
    __builtin_amdgcn_sched_barrier(0);                                                                      \
    if (++kt == ktc) {                                                                                      \
      /* readout of tile r: each 16-row x 32-column piece leaves in two stores of 8 whole */                \
      /* 128-byte lines: the upper 8 lanes of every 16-lane row trade their block-0 values */               \
      /* for block 1 of the lanes 8 below (DPP), so a lane then holds row lane%8 (+8 in the */              \
      /* second store) of the piece, columns 16*(lane/8%2) + 4*(lane/16)..+3 of the pair */                 \
      int tm, tn;                                                                                           \
      group_tile(c0 + slot + r * nslots, tiles_m, tiles_n, tm, tn);                                         \
      const float *par = (const float *)(params + (r & 1) * kFragBytes);                                    \
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(                                \
          y + (size_t)tm * BM * n, 0, (uint32_t)min(BM, m - tm * BM) * (uint32_t)n * 4u, 0x00020000);       \
      const uint32_t vcol = ((uint32_t)(lane & 7) * (uint32_t)n + (uint32_t)(tn * BN + wn * WTN + scol)) * 4u; \
      _Pragma("unroll") for (int jp = 0; jp < FN / 2; ++jp) {                                               \
        const hb_f32x4 b0 = has_bias ? *(const hb_f32x4 *)(par + lcol + jp * 32) : hb_f32x4{0, 0, 0, 0};    \
        const hb_f32x4 b1 = has_bias ? *(const hb_f32x4 *)(par + lcol + jp * 32 + 16) : hb_f32x4{0, 0, 0, 0}; \
        /* n % 32 == 0: a 32-column pair lies wholly inside or wholly past n */                            \
        if (tn * BN + wn * WTN + jp * 32 >= n) continue;                                                    \
        _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                                    \
          hb_u32x4 o0, o1, lo, hi;                                                                          \
          _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                                   \
            o0[e] = f16_out_bits<MODE>(acc[i][2 * jp][e], b0[e], has_bias);                                 \
            o1[e] = f16_out_bits<MODE>(acc[i][2 * jp + 1][e], b1[e], has_bias);                             \
          }                                                                                                 \
          _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                                   \
            lo[e] = (uint32_t)__builtin_amdgcn_update_dpp((int)o0[e], (int)o1[e], kDppRowShr8, 0xf, 0xc, false); \
            hi[e] = (uint32_t)__builtin_amdgcn_update_dpp((int)o1[e], (int)o0[e], kDppRowShl8, 0xf, 0x3, false); \
          }                                                                                                 \
          /* the whole offset in the vector operand: the range check that drops rows past m */              \
          /* does not cover the scalar offset */                                                             \
          const uint32_t srow = (uint32_t)(wm * WTM + i * 16) * (uint32_t)n * 4u;                            \
          __builtin_amdgcn_raw_buffer_store_b128(lo, rsrc, vcol + srow + (uint32_t)jp * 128u, 0, 2);        \
          __builtin_amdgcn_raw_buffer_store_b128(hi, rsrc, vcol + srow + (uint32_t)n * 32u + (uint32_t)jp * 128u, 0, 2); \
        }                                                                                                   \
      }                                                                                                     \
      _Pragma("unroll") for (int i = 0; i < FM; ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j)          \
          acc[i][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};                                                     \
      kt = 0;                                                                                               \
      ++r;                                                                                                  \
    }                                                                                                       \
  }

  for (int g = 0; g < steps; g += 2) {
    F16_STREAM_STEP(0)
    if (g + 1 < steps) F16_STREAM_STEP(1)
  }
#undef F16_STREAM_STEP
#undef F16_STREAM_MFMA
}

// ---------------------------------------------------------------------------
// Opcodes 8/10/11/12 with the post-processing in the GEMM epilogue: the ring
// kernel's 128 x BN tile (whole heads: BN = 192, three heads of 64; BN = 128,
// one head of 128 or two of 64; all of Q, K or V, since heads * HD is a
// multiple of BN) is read out to fp16 exactly as f16_gemm_ring reads it out
// (mode 0, no bias), kept in LDS as fp16 (the values are fp16-exact) instead
// of going to HBM as f32, and each (32-token tile, head) of it goes through
// qkv_block, the standalone post-processing kernel's code.  Results are
// identical to f16_gemm_ring followed by qkv_post.
// ---------------------------------------------------------------------------

template <int HD, int BN>
__global__ __launch_bounds__(256) void f16_qkv_ring(uint16_t *__restrict__ q, uint16_t *__restrict__ k,
                                                    uint16_t *__restrict__ v, const int8_t *__restrict__ aimg,
                                                    const int8_t *__restrict__ wpack, const float *__restrict__ bias,
                                                    const float *__restrict__ q_norm,
                                                    const float *__restrict__ k_norm, const float *__restrict__ pe,
                                                    int rope_off, int rope_count, int m, int kdim, int n_heads,
                                                    int token_tiles, int out_tile0) {
  constexpr int BM = 128, WM = 2, WN = 2, S = 4;
  static_assert(BN % HD == 0, "whole heads per tile");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int STAGE = (BM / 16 + BN / 16) * kFragBytes;
  constexpr int TS = BN + 8;  // halfwords per LDS row of the tile (padded)
  constexpr int TILE_BYTES = BM * TS * 2;
  constexpr int NH = BN / HD;                          // heads per tile, post-processed together
  constexpr int POST_BYTES = TILE_BYTES + NH * HD * 32 * 2;  // the tile, then its packed blocks
  static_assert(kQkvThreads == 64 * WM * WN, "the post-processing uses the GEMM's 256 threads");
  __shared__ __attribute__((aligned(1024))) int8_t lds[S * STAGE > POST_BYTES ? S * STAGE : POST_BYTES];
  uint16_t *blk = (uint16_t *)(lds + TILE_BYTES);

  const int q_cols = n_heads * HD, n = 3 * q_cols;
  const int tiles_m = (m + BM - 1) / BM, tiles_n = n / BN;
  int tm, tn;
  tile_coords_2d<BM, BN>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  hb_f32x4 acc[FM][FN];
  ring_mainloop<BM, BN, WM, WN, S>(acc, lds, aimg, wpack, m, kdim, n, m0, n0, wave, lane);

  block_barrier();  // every wave is done with the operand stages: LDS holds the tile
  _Float16 *tile = (_Float16 *)lds;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        tile[(wm * WTM + i * 16 + (lane >> 4) * 4 + r) * TS + wn * WTN + j * 16 + (lane & 15)] =
            (_Float16)acc[i][j][r];
  __syncthreads();

  const int which = n0 / q_cols, head0 = (n0 % q_cols) / HD;
  uint16_t *dst = which == 0 ? q : which == 1 ? k : v;
  const int rows_tile = min(BM, m - m0);
  const size_t head_stride = (size_t)token_tiles * (HD / 32) * 1024;
  for (int t = 0; t < BM / 32 && 32 * t < rows_tile; ++t) {
    const int rows = min(32, rows_tile - 32 * t);
    const int tt = out_tile0 + m0 / 32 + t;
    const size_t head_base = (size_t)head0 * head_stride;
    const _Float16 *src = tile + 32 * t * TS;
    const float *b = bias ? bias + n0 : nullptr;
    if (which == 0)
      qkv_blocks<HD, 0, NH>(blk, dst, src, TS, b, q_norm, pe, rope_off, rope_count, rows, m0 + 32 * t, tt,
                            token_tiles, head_base, head_stride);
    else if (which == 1)
      qkv_blocks<HD, 1, NH>(blk, dst, src, TS, b, k_norm, pe, rope_off, rope_count, rows, m0 + 32 * t, tt,
                            token_tiles, head_base, head_stride);
    else
      qkv_blocks<HD, 2, NH>(blk, dst, src, TS, b, nullptr, nullptr, 0, 0, rows, m0 + 32 * t, tt, token_tiles,
                            head_base, head_stride);
    __syncthreads();  // the packed blocks' LDS staging is reused by the next token tile
  }
}

// ---------------------------------------------------------------------------
// Few rows (m <= 128): split-K.  Workgroup (g, s) computes all rows x 32
// columns (col-group g) over the s-th range of 32-k blocks; its 4 waves take
// the range's blocks round robin and are summed in LDS in wave order, then
// the partial tile goes to workspace slice s.  A second kernel sums the
// slices in order (so results do not depend on scheduling), rounds to fp16
// (the readout step) and applies bias and activation.  Operands are read
// straight from memory in MFMA lane order: W from the packed image (one 1 KB
// tile per 16 columns x 32 k), A as 8 fp32 per lane converted to fp16 (RNE).
// ---------------------------------------------------------------------------

constexpr int kSkinnyWaves = 4;

// RF row fragments (16 rows each) x CF column fragments per workgroup; each
// wave owns KPW consecutive 32-k blocks of the split, whose operands it
// requests all at once before the first MFMA.
template <int RF, int CF, int KPW>
__global__ __launch_bounds__(64 * kSkinnyWaves) void f16_skinny_partial(float *__restrict__ ws,
                                                                        const float *__restrict__ x,
                                                                        const uint16_t *__restrict__ packed, int m,
                                                                        int k, int n) {
  __shared__ hb_f32x4 red[kSkinnyWaves - 1][RF * CF][64];
  const int g = blockIdx.x, s = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kblocks = k / 32;
  const int kb0 = (s * kSkinnyWaves + wave) * KPW;
  // operands (block indices clamped into range; blocks past the end are not multiplied)
  hb_f16x8 b[KPW][CF];
  float4 alo[KPW][RF], ahi[KPW][RF];
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    const int kb = min(kb0 + t, kblocks - 1);
#pragma unroll
    for (int j = 0; j < CF; ++j)
      b[t][j] = *(const hb_f16x8 *)(packed + ((size_t)(g * CF + j) * kblocks + kb) * 512u + lane * 8);
#pragma unroll
    for (int i = 0; i < RF; ++i) {
      const float *xr = x + (size_t)min(16 * i + (lane & 15), m - 1) * k + kb * 32 + 8 * (lane >> 4);
      alo[t][i] = *(const float4 *)xr;
      ahi[t][i] = *(const float4 *)(xr + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first use
  hb_f32x4 acc[RF][CF];
#pragma unroll
  for (int i = 0; i < RF; ++i)
#pragma unroll
    for (int j = 0; j < CF; ++j) acc[i][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    if (kb0 + t < kblocks) {
#pragma unroll
      for (int i = 0; i < RF; ++i) {
        const hb_f16x8 a = {(_Float16)alo[t][i].x, (_Float16)alo[t][i].y, (_Float16)alo[t][i].z,
                            (_Float16)alo[t][i].w, (_Float16)ahi[t][i].x, (_Float16)ahi[t][i].y,
                            (_Float16)ahi[t][i].z, (_Float16)ahi[t][i].w};
        // W as the A operand: lane l holds 4 consecutive columns of row l % 16
#pragma unroll
        for (int j = 0; j < CF; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[t][j], a, acc[i][j], 0, 0, 0);
      }
    }
  }
  if (wave != 0) {
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int j = 0; j < CF; ++j) red[wave - 1][i * CF + j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave != 0) return;
  // 16-byte stores through a buffer resource covering the slice's first m
  // rows: rows past m are never read and fall outside it (dropped, no branches)
  const int mp = (m + 15) / 16 * 16;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(ws + (size_t)s * mp * n, 0, m * n * 4, 0x00020000);
#pragma unroll
  for (int i = 0; i < RF; ++i) {
#pragma unroll
    for (int j = 0; j < CF; ++j) {
      hb_f32x4 t = acc[i][j];
#pragma unroll
      for (int w = 1; w < kSkinnyWaves; ++w) t += red[w - 1][i * CF + j][lane];
      const int row = 16 * i + (lane & 15), col = (g * CF + j) * 16 + 4 * (lane >> 4);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(hb_u32x4, t), rs, (uint32_t)(row * n + col) * 4u, 0,
                                             0);
    }
  }
}

// ---------------------------------------------------------------------------
// Few rows on quantized weights (opcodes 2/3/4, m <= 16): the split-K kernel
// above with the weight fragment built from the super-blocks themselves, so
// a call streams 4.5 (Q4_0, IQ4_NL) or 8.5 (Q8_0) bits per weight instead of
// the 16 of the F16 image.  Fragment (16 columns gc, 32-k block kb), lane l:
// column c = (gc%2)*16 + l%16 of 32-column tile gc/2, super-block q = l/16 of
// the tile's k-block (8 k x 32 columns).  Its 8 values k = 2p+e (p < 4, e < 2)
// sit, for Q4_0 / IQ4_NL, in the nibbles of quant word c (bytes 4c..4c+3):
// pair p takes bytes (0,2), (1,3) low nibbles for p = 0, 1 and high nibbles
// for p = 2, 3 (the vlut16 order of qk0_prepack, rewritten for one column);
// for Q8_0 in the byte pair at 64p + 2c.  Scale of pair p: s[2p + c/16].
// Values become fp16 exactly (1024 + biased code in the mantissa, minus the
// bias) and one packed fp16 multiply rounds value*scale as qk0_prepack does,
// so the result equals hb_f16_gemm_ws on the prepacked image bit for bit.
// ---------------------------------------------------------------------------

typedef _Float16 hb_f16x2 __attribute__((ext_vector_type(2)));

template <int TYPE>
struct Qk0Raw {
  uint32_t q[TYPE == HB_GGML_Q8_0 ? 4 : 1];
  hb_u32x4 s;  // the super-block's 8 fp16 scales
};

template <int TYPE>
constexpr int qk0_block_bytes() {
  return TYPE == HB_GGML_Q8_0 ? 272 : 144;
}

template <int TYPE>
__device__ inline void qk0_load(Qk0Raw<TYPE> &r, const uint8_t *__restrict__ blocks, int gc, int kb, int kblocks,
                                int lane) {
  const int c = (gc & 1) * 16 + (lane & 15), q = lane >> 4;
  const uint8_t *base = blocks + ((size_t)((gc >> 1) * kblocks + kb) * 4u + (size_t)q) * (size_t)qk0_block_bytes<TYPE>();
  r.s = *(const hb_u32x4 *)base;
  if constexpr (TYPE == HB_GGML_Q8_0) {
#pragma unroll
    for (int p = 0; p < 4; ++p) r.q[p] = __builtin_nontemporal_load((const uint16_t *)(base + 16 + 64 * p + 2 * c));
  } else {
    r.q[0] = __builtin_nontemporal_load((const uint32_t *)(base + 16 + 4 * c));
  }
}

// IQ4_NL code book + 128, as bytes (ggml's kvalues_iq4nl).
constexpr uint32_t kIq4Biased[4] = {0x3F2D1801u, 0x766A5D4Fu, 0xA6998D81u, 0xF1D9C5B5u};

// Four nibbles (one per byte) -> their biased IQ4_NL codes: two byte
// permutes look up the low and high halves of the code book, bit 3 of each
// nibble picks one (v_bfi).
__device__ inline uint32_t iq4_lookup(uint32_t nib) {
  const uint32_t sel = nib & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIq4Biased[1], kIq4Biased[0], sel);
  const uint32_t hi = __builtin_amdgcn_perm(kIq4Biased[3], kIq4Biased[2], sel);
  const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}

// The 8 fp16 weights a lane holds of one fragment.  Pair p's two codes go
// into the low bytes of an fp16 pair whose high bytes are 0x64 (the value
// 1024 + code, exact), one packed subtract of the bias leaves the exact
// code, one packed multiply by the pair's scale rounds code * scale once.
// The byte moves are single permutes where the codes are whole bytes and an
// and-or where they are nibbles (Q4_0); the scale of pair p (low or high
// half of scale word p) is broadcast to both halves by one permute.
template <int TYPE>
__device__ inline hb_f16x8 qk0_fragment(const Qk0Raw<TYPE> &r, int odd) {
  constexpr uint32_t kExp = 0x64646464u;  // permute source of the 0x64 high bytes (selector 4)
  uint32_t u[4];  // pair p: 0x64 | code0, 0x64 | code1
  float bias;
  if constexpr (TYPE == HB_GGML_Q8_0) {
    // int8 codes: +128 by flipping bit 7 (the 0x64 bytes are untouched)
#pragma unroll
    for (int p = 0; p < 4; ++p) u[p] = __builtin_amdgcn_perm(kExp, r.q[p], 0x04010400u) ^ 0x00800080u;
    bias = 1152.0f;
  } else if constexpr (TYPE == HB_GGML_IQ4_NL) {
    // pair p takes bytes (0,2), (1,3) of the low nibbles' codes for p = 0, 1, of the high for p = 2, 3
    const uint32_t lo = iq4_lookup(r.q[0] & 0x0F0F0F0Fu), hi = iq4_lookup((r.q[0] >> 4) & 0x0F0F0F0Fu);
    u[0] = __builtin_amdgcn_perm(kExp, lo, 0x04020400u);
    u[1] = __builtin_amdgcn_perm(kExp, lo, 0x04030401u);
    u[2] = __builtin_amdgcn_perm(kExp, hi, 0x04020400u);
    u[3] = __builtin_amdgcn_perm(kExp, hi, 0x04030401u);
    bias = 1152.0f;
  } else {
    // Q4_0: pair p takes the low nibbles of bytes (0,2), (1,3) for p = 0, 1,
    // the high nibbles for p = 2, 3
    // (one v_and_or_b32 each; gfx9 VOP3 takes no literal, so the mask comes
    // from an SGPR and the exponent bytes from a VGPR)
    const uint32_t w = r.q[0];
    const uint32_t nib = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    uint32_t e = 0x64006400u;
    asm("" : "+v"(e));  // keep the exponent bytes in a VGPR
    const uint32_t src[4] = {w, w >> 8, w >> 4, w >> 12};
#pragma unroll
    for (int p = 0; p < 4; ++p) asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(u[p]) : "v"(src[p]), "s"(nib), "v"(e));
    bias = 1032.0f;
  }
  const hb_f16x2 b2 = {(_Float16)bias, (_Float16)bias};
  const uint32_t ssel = odd ? 0x03020302u : 0x01000100u;
  hb_u32x4 out;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // the scale of pair p, broadcast to both halves by one permute (a vector
    // shuffle of the extracted word here was compiled to the multiply's
    // operand selection on scale word 0 for every p: wrong results)
    const hb_f16x2 sc = __builtin_bit_cast(hb_f16x2, __builtin_amdgcn_perm(r.s[p], r.s[p], ssel));
    const hb_f16x2 v = __builtin_bit_cast(hb_f16x2, u[p]) - b2;  // exact codes
    out[p] = __builtin_bit_cast(uint32_t, v * sc);                 // one fp16 rounding of code * scale
  }
  return __builtin_bit_cast(hb_f16x8, out);
}

// One row (m == 1) on quantized weights: one workgroup per 32-column tile,
// WAVES waves each owning KB consecutive 32-k blocks of the whole K, so the
// tile is finished in one launch with no partial sums in memory.  Every wave
// first requests all its quant words and scales, the workgroup meanwhile
// converts the row to fp16 into LDS (in the A-operand order: only lanes of
// row 0, lane % 16 == 0, carry it), then the fragments are dequantized and
// multiplied; the waves' sums are added in wave order in LDS before the fp16
// readout.
template <int TYPE, int WAVES, int KB, int BT>
__global__ __launch_bounds__(64 * WAVES) void qk0_decode(float *__restrict__ y, const float *__restrict__ x,
                                                        const uint8_t *__restrict__ blocks, int k, int n) {
  static_assert(KB % BT == 0, "k-blocks per wave must split into batches");
  constexpr int NB = KB / BT;                          // batches per wave
  constexpr int XV = (WAVES * KB * 8) / (64 * WAVES);  // float4 of the row per thread
  __shared__ __attribute__((aligned(16))) _Float16 xs[WAVES * KB * 32];
  __shared__ float red[WAVES][32];
  const int tile = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kblocks = k / 32;
  const int kb0 = wave * KB;
  // the row first (oldest loads: waiting for it leaves the weights in flight)
  float4 xv[XV];
#pragma unroll
  for (int i = 0; i < XV; ++i) xv[i] = *(const float4 *)(x + 4 * min((int)threadIdx.x + 64 * WAVES * i, k / 4 - 1));
  Qk0Raw<TYPE> raw[KB][2];
  auto issue = [&](int b) {
#pragma unroll
    for (int t = b * BT; t < b * BT + BT; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        qk0_load<TYPE>(raw[t][j], blocks, 2 * tile + j, min(kb0 + t, kblocks - 1), kblocks, lane);
  };
  issue(0);
  if (NB > 1) issue(1);
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int v = threadIdx.x + 64 * WAVES * i;
    // unconditional use of the loads (a conditional one lets the compiler
    // move them into a branch, behind a wait for every weight request)
    xs[4 * v] = (_Float16)xv[i].x;
    xs[4 * v + 1] = (_Float16)xv[i].y;
    xs[4 * v + 2] = (_Float16)xv[i].z;
    xs[4 * v + 3] = (_Float16)xv[i].w;
    if (4 * v >= k) *(uint2 *)(xs + 4 * v) = make_uint2(0u, 0u);  // zeros past k
  }
  __syncthreads();
  const bool has_row = (lane & 15) == 0;
  hb_f32x4 acc[2] = {hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f}, hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
  // Batch b is multiplied while batches b+1 and b+2 are in flight.  No
  // branches around the multiplies (a branch would let the compiler sink the
  // loads into it): k-blocks past k multiply zero weights by the zero row.
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b + 2 < NB) issue(b + 2);
#pragma unroll
    for (int t = b * BT; t < b * BT + BT; ++t) {
      const int kb = kb0 + t;
      const bool live = kb < kblocks;
      const hb_f16x8 a = has_row ? *(const hb_f16x8 *)(xs + kb * 32 + 8 * (lane >> 4)) : hb_f16x8{};
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const hb_f16x8 w = live ? qk0_fragment<TYPE>(raw[t][j], j) : hb_f16x8{};
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, a, acc[j], 0, 0, 0);
      }
    }
  }
  // row 0 of the product: element r of lanes 0, 16, 32, 48 holds column 4*(lane/16) + r
  if (has_row) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][16 * j + 4 * (lane >> 4) + r] = acc[j][r];
  }
  __syncthreads();
  if (threadIdx.x >= 32) return;
  float sum = red[0][threadIdx.x];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) sum += red[w][threadIdx.x];
  y[tile * 32 + threadIdx.x] = (float)(_Float16)sum;
}

// One row (m == 1) on quantized weights, the weights streamed through LDS:
// the same plan as qk0_decode (a workgroup per 32-column tile; wave w owns
// k-blocks [w*KB, w*KB + KB), whose 4 super-blocks each lie back to back,
// so a wave's weights are one contiguous run of KB * 4 * block bytes), but
// the run arrives in whole 1 KB pieces (buffer_load ... lds, 16 bytes per
// lane) into a 4 KB ring per wave instead of 2- to 16-byte register loads
// per lane, which moved up to four times the run's bytes through the CU's
// memory pipeline (every lane of a super-block fetched its 16 scale bytes).
// A piece is re-used for the ring once every fragment that reads it has
// been multiplied; the fragments are dequantized from LDS exactly as from
// registers (qk0_fragment), so the arithmetic is qk0_decode's.
template <int TYPE, int WAVES, int KB>
__global__ __launch_bounds__(64 * WAVES) void qk0_decode_ring(float *__restrict__ y, const float *__restrict__ x,
                                                             const uint8_t *__restrict__ blocks, int k, int n) {
  constexpr int BB = qk0_block_bytes<TYPE>(), BLK = 4 * BB;  // bytes of one 32-k block of a tile
  constexpr int RUN = KB * BLK, NCH = (RUN + 1023) / 1024, RS = 4;
  constexpr int XV = (WAVES * KB * 8) / (64 * WAVES);  // float4 of the row per thread
  __shared__ __attribute__((aligned(1024))) uint8_t ring[WAVES][RS * 1024];
  __shared__ __attribute__((aligned(16))) _Float16 xs[WAVES * KB * 32];
  __shared__ float red[WAVES][32];
  const int tile = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kblocks = k / 32;
  const int kb0 = wave * KB;
  // the row first (its registers are needed before any weight arrives)
  float4 xv[XV];
#pragma unroll
  for (int i = 0; i < XV; ++i) xv[i] = *(const float4 *)(x + 4 * min((int)threadIdx.x + 64 * WAVES * i, k / 4 - 1));
  // this wave's run, piece by piece (global_load_lds: the compiler then tracks
  // which LDS bytes each piece writes, so reading a landed piece does not wait
  // for the later ones).  Addresses past the weights are clamped to their
  // last 16 bytes; those bytes, like other tiles' blocks read past a short K,
  // are never multiplied.
  const size_t total = (size_t)(n / 32) * (size_t)kblocks * (size_t)BLK;
  const size_t run0 = ((size_t)tile * (size_t)kblocks + (size_t)kb0) * (size_t)BLK;
  uint8_t *const mine = ring[wave];
  const uint32_t ring_lds = (uint32_t)(uintptr_t)HB_LDS_PTR(mine);  // LDS address of this wave's ring
  auto piece = [&](int c) {
    const size_t off = min(run0 + (size_t)c * 1024u + (size_t)lane * 16u, total - 16u);
    __builtin_amdgcn_global_load_lds(blocks + off, HB_LDS_PTR(mine + (c % RS) * 1024), 16, 0, 0);
  };
  // The row goes to LDS before any weight piece is requested: pieces
  // requested first (by every workgroup at once) queue ahead of the rows in
  // the memory system and held a workgroup's row back for about 3 us
  // (phase stamps), with its ring full and nothing to multiply.
#pragma unroll
  for (int i = 0; i < XV; ++i) {
    const int v = threadIdx.x + 64 * WAVES * i;
    xs[4 * v] = (_Float16)xv[i].x;
    xs[4 * v + 1] = (_Float16)xv[i].y;
    xs[4 * v + 2] = (_Float16)xv[i].z;
    xs[4 * v + 3] = (_Float16)xv[i].w;
    if (4 * v >= k) *(uint2 *)(xs + 4 * v) = make_uint2(0u, 0u);  // zeros past k
  }
#pragma unroll
  for (int c = 0; c < RS && c < NCH; ++c) piece(c);
  // the row in LDS for every wave (a bare barrier: __syncthreads would also
  // wait for the pieces in flight)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  block_barrier();
  const bool has_row = (lane & 15) == 0;
  const int q = lane >> 4, c16 = lane & 15;
  hb_f32x4 acc[2] = {hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f}, hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
  int issued = RS < NCH ? RS : NCH;
#pragma unroll
  for (int t = 0; t < KB; ++t) {
    // every piece of k-block t has landed: at most (issued - 1 - last) younger pieces outstanding
    const int last = (t * BLK + BLK - 1) / 1024;
    switch (issued - 1 - last) {
      case 0: wait_vmcnt<0>(); break;
      case 1: wait_vmcnt<1>(); break;
      case 2: wait_vmcnt<2>(); break;
      default: wait_vmcnt<3>(); break;
    }
    const int kb = kb0 + t;
    const bool live = kb < kblocks;
    // every lane reads row 0's values: the other lanes' A values reach only
    // rows 1-15 of the product, which are never read
    const hb_f16x8 a = *(const hb_f16x8 *)(xs + kb * 32 + 8 * (lane >> 4));
    // this lane's super-block in the ring.  The reads are written as LDS
    // instructions the compiler does not track: it cannot tell them from the
    // pieces still in flight into the ring, and would wait for every one of
    // them (vmcnt(0)) before each read; the wait above covers the bytes read.
    const int sb = (t * BLK + q * BB) % (RS * 1024);
    Qk0Raw<TYPE> raw[2];
    hb_u32x4 scales;
    asm volatile("ds_read_b128 %0, %1" : "=v"(scales) : "v"(ring_lds + (uint32_t)sb));
    uint32_t codes[2][TYPE == HB_GGML_Q8_0 ? 4 : 1];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = j * 16 + c16;
      if constexpr (TYPE == HB_GGML_Q8_0) {
#pragma unroll
        for (int p = 0; p < 4; ++p)
          asm volatile("ds_read_u16 %0, %1"
                       : "=v"(codes[j][p])
                       : "v"(ring_lds + (uint32_t)((sb + 16 + 64 * p + 2 * c) % (RS * 1024))));
      } else {
        asm volatile("ds_read_b32 %0, %1" : "=v"(codes[j][0]) : "v"(ring_lds + (uint32_t)((sb + 16 + 4 * c) % (RS * 1024))));
      }
    }
    // the values are used only after this wait (they pass through it)
    if constexpr (TYPE == HB_GGML_Q8_0)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(scales), "+v"(codes[0][0]), "+v"(codes[0][1]), "+v"(codes[0][2]), "+v"(codes[0][3]),
                     "+v"(codes[1][0]), "+v"(codes[1][1]), "+v"(codes[1][2]), "+v"(codes[1][3]));
    else
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(scales), "+v"(codes[0][0]), "+v"(codes[1][0]));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      raw[j].s = scales;
#pragma unroll
      for (int p = 0; p < (TYPE == HB_GGML_Q8_0 ? 4 : 1); ++p) raw[j].q[p] = codes[j][p];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const hb_f16x8 w = live ? qk0_fragment<TYPE>(raw[j], j) : hb_f16x8{};
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, a, acc[j], 0, 0, 0);
    }
    // pieces before k-block t + 1's first are free once these reads are done
    const int next_first = t + 1 < KB ? ((t + 1) * BLK) / 1024 : NCH;
    if (issued < NCH && issued < next_first + RS) {
      __builtin_amdgcn_sched_barrier(0);  // (the reads of the freed pieces completed at the wait above)
      while (issued < NCH && issued < next_first + RS) piece(issued++);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // row 0 of the product: element r of lanes 0, 16, 32, 48 holds column 4*(lane/16) + r
  if (has_row) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][16 * j + 4 * (lane >> 4) + r] = acc[j][r];
  }
  __syncthreads();
  if (threadIdx.x >= 32) return;
  float sum = red[0][threadIdx.x];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) sum += red[w][threadIdx.x];
  y[tile * 32 + threadIdx.x] = (float)(_Float16)sum;
}

// 2 to 16 rows on the one-row kernel's plan, 64 columns per workgroup: wave
// w streams the runs of k-blocks [KB*w, KB*w + KB) of both 32-column tiles
// of its workgroup through two LDS rings (piece c of both runs requested
// together), so a workgroup reads each activation value once for 64 columns
// and the 224 workgroups of N = 14336 take one round of the CUs.  Each wave
// owns a k-range and loads only that range of the rows: lane l's share of
// activation row l % 16 (eight values per k-block; rows past m repeat row
// m - 1 and are never stored), requested before any weight piece so that
// every piece wait also covers them.  The waves' 16 x 64 partial products
// are added in wave order in LDS (the rings, free by then), then read out to
// fp16.  n % 64 == 0.
template <int TYPE, int WAVES, int KB>
__global__ __launch_bounds__(64 * WAVES) void qk0_rows_ring(float *__restrict__ y, const float *__restrict__ x,
                                                           const uint8_t *__restrict__ blocks, int m, int k, int n) {
  constexpr int BB = qk0_block_bytes<TYPE>(), BLK = 4 * BB;  // bytes of one 32-k block of a 32-column tile
  constexpr int RUN = KB * BLK, NCH = (RUN + 1023) / 1024, RS = 4;
  constexpr int NQ = TYPE == HB_GGML_Q8_0 ? 4 : 1;  // code words per fragment
  __shared__ __attribute__((aligned(1024))) uint8_t ring[WAVES][2][RS * 1024];
  static_assert(WAVES == 16, "one output value per thread: 16 rows x 64 columns");
  static_assert(sizeof(ring) >= WAVES * 1024 * sizeof(float), "the partial products fit in the rings");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kblocks = k / 32;
  const int kb0 = wave * KB;
  // this wave's k-range of the rows (blocks past k repeat the last one and are not multiplied)
  const float *xr = x + (size_t)min(lane & 15, m - 1) * (size_t)k + 8 * (lane >> 4);
  float4 alo[KB], ahi[KB];
#pragma unroll
  for (int t = 0; t < KB; ++t) {
    const int kb = min(kb0 + t, kblocks - 1);
    alo[t] = *(const float4 *)(xr + kb * 32);
    ahi[t] = *(const float4 *)(xr + kb * 32 + 4);
  }
  const size_t total = (size_t)(n / 32) * (size_t)kblocks * (size_t)BLK;
  size_t run0[2];
  uint32_t ring_lds[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    run0[r] = ((size_t)(2 * blockIdx.x + r) * (size_t)kblocks + (size_t)kb0) * (size_t)BLK;
    ring_lds[r] = (uint32_t)(uintptr_t)HB_LDS_PTR(ring[wave][r]);
  }
  auto pieces = [&](int c) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const size_t off = min(run0[r] + (size_t)c * 1024u + (size_t)lane * 16u, total - 16u);
      __builtin_amdgcn_global_load_lds(blocks + off, HB_LDS_PTR(ring[wave][r] + (c % RS) * 1024), 16, 0, 0);
    }
  };
#pragma unroll
  for (int c = 0; c < RS && c < NCH; ++c) pieces(c);
  const int q = lane >> 4, c16 = lane & 15;
  hb_f32x4 acc[2][2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[r][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  int issued = RS < NCH ? RS : NCH;
#pragma unroll
  for (int t = 0; t < KB; ++t) {
    // piece `last` of both runs has landed (and every row load, requested
    // before the pieces): at most two younger pieces per later index
    const int last = (t * BLK + BLK - 1) / 1024;
    switch (issued - 1 - last) {
      case 0: wait_vmcnt<0>(); break;
      case 1: wait_vmcnt<2>(); break;
      case 2: wait_vmcnt<4>(); break;
      default: wait_vmcnt<6>(); break;
    }
    const bool live = kb0 + t < kblocks;
    const hb_f16x8 a = live ? hb_f16x8{(_Float16)alo[t].x, (_Float16)alo[t].y, (_Float16)alo[t].z,
                                       (_Float16)alo[t].w, (_Float16)ahi[t].x, (_Float16)ahi[t].y,
                                       (_Float16)ahi[t].z, (_Float16)ahi[t].w}
                            : hb_f16x8{};
    // LDS reads the compiler does not track, as in the one-row kernel
    const int sb = (t * BLK + q * BB) % (RS * 1024);
    hb_u32x4 scales[2];
    uint32_t codes[2][2][NQ];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      asm volatile("ds_read_b128 %0, %1" : "=v"(scales[r]) : "v"(ring_lds[r] + (uint32_t)sb));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = j * 16 + c16;
        if constexpr (TYPE == HB_GGML_Q8_0) {
#pragma unroll
          for (int p = 0; p < 4; ++p)
            asm volatile("ds_read_u16 %0, %1"
                         : "=v"(codes[r][j][p])
                         : "v"(ring_lds[r] + (uint32_t)((sb + 16 + 64 * p + 2 * c) % (RS * 1024))));
        } else {
          asm volatile("ds_read_b32 %0, %1"
                       : "=v"(codes[r][j][0])
                       : "v"(ring_lds[r] + (uint32_t)((sb + 16 + 4 * c) % (RS * 1024))));
        }
      }
    }
    if constexpr (TYPE == HB_GGML_Q8_0)
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(scales[0]), "+v"(scales[1]), "+v"(codes[0][0][0]), "+v"(codes[0][0][1]),
                     "+v"(codes[0][0][2]), "+v"(codes[0][0][3]), "+v"(codes[0][1][0]), "+v"(codes[0][1][1]),
                     "+v"(codes[0][1][2]), "+v"(codes[0][1][3]), "+v"(codes[1][0][0]), "+v"(codes[1][0][1]),
                     "+v"(codes[1][0][2]), "+v"(codes[1][0][3]), "+v"(codes[1][1][0]), "+v"(codes[1][1][1]),
                     "+v"(codes[1][1][2]), "+v"(codes[1][1][3]));
    else
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(scales[0]), "+v"(scales[1]), "+v"(codes[0][0][0]), "+v"(codes[0][1][0]),
                     "+v"(codes[1][0][0]), "+v"(codes[1][1][0]));
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        Qk0Raw<TYPE> raw;
        raw.s = scales[r];
#pragma unroll
        for (int p = 0; p < NQ; ++p) raw.q[p] = codes[r][j][p];
        const hb_f16x8 w = live ? qk0_fragment<TYPE>(raw, j) : hb_f16x8{};
        acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, a, acc[r][j], 0, 0, 0);
      }
    const int next_first = t + 1 < KB ? ((t + 1) * BLK) / 1024 : NCH;
    if (issued < NCH && issued < next_first + RS) {
      __builtin_amdgcn_sched_barrier(0);
      while (issued < NCH && issued < next_first + RS) pieces(issued++);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // every piece has been waited for and every ring read is done once all
  // waves pass the barrier: the rings hold the partial products, [wave][1024]
  __syncthreads();
  float *red = (float *)&ring[0][0][0];
  // lane l holds row l % 16, columns 32*r + 16*j + 4*(l/16) + e
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave * 1024 + (r * 2 + j) * 256 + e * 64 + lane] = acc[r][j][e];
  __syncthreads();
  const int i = threadIdx.x, l = i & 63;  // one output value per thread
  const int row = l & 15;
  if (row >= m) return;
  float sum = red[i];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) sum += red[w * 1024 + i];
  const int col = blockIdx.x * 64 + 16 * (i >> 8) + 4 * (l >> 4) + ((i >> 6) & 3);
  y[(size_t)row * n + col] = (float)(_Float16)sum;
}

template <int RF, int CF, int KPW, int TYPE>
__global__ __launch_bounds__(64 * kSkinnyWaves) void qk0_skinny_partial(float *__restrict__ ws,
                                                                        const float *__restrict__ x,
                                                                        const uint8_t *__restrict__ blocks, int m,
                                                                        int k, int n) {
  __shared__ hb_f32x4 red[kSkinnyWaves - 1][RF * CF][64];
  const int g = blockIdx.x, s = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kblocks = k / 32;
  const int kb0 = (s * kSkinnyWaves + wave) * KPW;
  Qk0Raw<TYPE> raw[KPW][CF];
  float4 alo[KPW][RF], ahi[KPW][RF];
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    const int kb = min(kb0 + t, kblocks - 1);
#pragma unroll
    for (int j = 0; j < CF; ++j) qk0_load<TYPE>(raw[t][j], blocks, g * CF + j, kb, kblocks, lane);
#pragma unroll
    for (int i = 0; i < RF; ++i) {
      const float *xr = x + (size_t)min(16 * i + (lane & 15), m - 1) * k + kb * 32 + 8 * (lane >> 4);
      alo[t][i] = *(const float4 *)xr;
      ahi[t][i] = *(const float4 *)(xr + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first use
  hb_f32x4 acc[RF][CF];
#pragma unroll
  for (int i = 0; i < RF; ++i)
#pragma unroll
    for (int j = 0; j < CF; ++j) acc[i][j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    if (kb0 + t < kblocks) {
      hb_f16x8 b[CF];
#pragma unroll
      for (int j = 0; j < CF; ++j) b[j] = qk0_fragment<TYPE>(raw[t][j], (g * CF + j) & 1);
#pragma unroll
      for (int i = 0; i < RF; ++i) {
        const hb_f16x8 a = {(_Float16)alo[t][i].x, (_Float16)alo[t][i].y, (_Float16)alo[t][i].z,
                            (_Float16)alo[t][i].w, (_Float16)ahi[t][i].x, (_Float16)ahi[t][i].y,
                            (_Float16)ahi[t][i].z, (_Float16)ahi[t][i].w};
#pragma unroll
        for (int j = 0; j < CF; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[j], a, acc[i][j], 0, 0, 0);
      }
    }
  }
  if (wave != 0) {
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int j = 0; j < CF; ++j) red[wave - 1][i * CF + j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave != 0) return;
  // 16-byte stores through a buffer resource covering the slice's first m
  // rows: rows past m are never read and fall outside it (dropped, no branches)
  const int mp = (m + 15) / 16 * 16;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(ws + (size_t)s * mp * n, 0, m * n * 4, 0x00020000);
#pragma unroll
  for (int i = 0; i < RF; ++i) {
#pragma unroll
    for (int j = 0; j < CF; ++j) {
      hb_f32x4 t = acc[i][j];
#pragma unroll
      for (int w = 1; w < kSkinnyWaves; ++w) t += red[w - 1][i * CF + j][lane];
      const int row = 16 * i + (lane & 15), col = (g * CF + j) * 16 + 4 * (lane >> 4);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(hb_u32x4, t), rs, (uint32_t)(row * n + col) * 4u, 0,
                                             0);
    }
  }
}

// ---------------------------------------------------------------------------
// Small GEMMs (few rows, K <= W*KPW*32): one workgroup per 16 rows x 16*CF
// columns over the whole K.  Its W waves split K, each requesting all of its
// operands (KPW 32-k blocks of x and of CF weight tiles) before the first
// multiply, so a workgroup pays one memory latency; the waves' sums are added
// in LDS in wave order (deterministic), then the fp16 readout, bias and
// activation, and 16-byte row stores (or the channel-major store of mode 3).
// One launch, no workspace.  Weights are the MFMA A operand, as in the
// split-K kernel: lane l holds 4 consecutive columns of row l % 16.
// ---------------------------------------------------------------------------

// TYPE 0: weights are the packed fp16 image; HB_GGML_*: quantized
// super-blocks, each fragment dequantized in registers as in qk0_skinny_partial
// (the same fp16 values, so both forms give the same bits).
template <int CF, int W, int KPW, int TYPE>
__global__ __launch_bounds__(64 * W) void f16_small(float *__restrict__ y, const float *__restrict__ x,
                                                   const void *__restrict__ weights, const float *__restrict__ bias,
                                                   int m, int k, int n, int channels, int mode) {
  __shared__ hb_f32x4 red[W][CF][64];
  const int rt = blockIdx.x, g = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kblocks = k / 32;
  const int kb0 = wave * KPW;
  const int row = rt * 16 + (lane & 15);
  const float *xr = x + (size_t)min(row, m - 1) * k + 8 * (lane >> 4);
  using Raw = typename std::conditional<TYPE == 0, hb_f16x8, Qk0Raw<TYPE == 0 ? HB_GGML_Q4_0 : TYPE>>::type;
  Raw b[KPW][CF];
  float4 alo[KPW], ahi[KPW];
  // the bias of the fragment this wave finishes (waves below CF), requested
  // with the operands
  const int col = (g * CF + (wave < CF ? wave : 0)) * 16 + 4 * (lane >> 4);
  float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (wave < CF && bias) {
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = col + r < channels ? bias[col + r] : 0.0f;
  }
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    const int kb = min(kb0 + t, kblocks - 1);  // blocks past k are loaded, then zeroed
#pragma unroll
    for (int j = 0; j < CF; ++j) {
      if constexpr (TYPE == 0)
        b[t][j] = *(const hb_f16x8 *)((const uint16_t *)weights + ((size_t)(g * CF + j) * kblocks + kb) * 512u +
                                      lane * 8);
      else
        qk0_load<TYPE>(b[t][j], (const uint8_t *)weights, g * CF + j, kb, kblocks, lane);
    }
    alo[t] = *(const float4 *)(xr + kb * 32);
    ahi[t] = *(const float4 *)(xr + kb * 32 + 4);
  }
  hb_f32x4 acc[CF];
#pragma unroll
  for (int j = 0; j < CF; ++j) acc[j] = hb_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < KPW; ++t) {
    const bool live = kb0 + t < kblocks;
    const hb_f16x8 a = live ? hb_f16x8{(_Float16)alo[t].x, (_Float16)alo[t].y, (_Float16)alo[t].z,
                                       (_Float16)alo[t].w, (_Float16)ahi[t].x, (_Float16)ahi[t].y,
                                       (_Float16)ahi[t].z, (_Float16)ahi[t].w}
                            : hb_f16x8{};
#pragma unroll
    for (int j = 0; j < CF; ++j) {
      hb_f16x8 w;
      if constexpr (TYPE == 0)
        w = b[t][j];
      else
        w = qk0_fragment<TYPE>(b[t][j], (g * CF + j) & 1);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, a, acc[j], 0, 0, 0);
    }
  }
#pragma unroll
  for (int j = 0; j < CF; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  // one output fragment per wave (CF <= W): rows of lane % 16, 4 columns
  if (wave >= CF || row >= m) return;
  const int j = wave;
  hb_f32x4 tot = red[0][j][lane];
#pragma unroll
  for (int w = 1; w < W; ++w) tot += red[w][j][lane];
  hb_f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = (float)(_Float16)tot[r];
    out[r] = bias && col + r < channels ? __fadd_rn(v, bv[r]) : v;
  }
  if (mode == 3) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (col + r < channels) y[(size_t)(col + r) * m + row] = out[r];
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] = apply_mode(out[r], mode);
    *(hb_f32x4 *)(y + (size_t)row * n + col) = out;
  }
}

__global__ __launch_bounds__(256) void f16_skinny_epilogue(float *__restrict__ y, const float *__restrict__ ws,
                                                          const float *__restrict__ bias, int m, int n,
                                                          int channels, int mode, int splits) {
  const int limit = mode == 3 ? channels : n;
  const size_t total = (size_t)m * limit;
  const int mp = (m + 15) / 16 * 16;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const int row = (int)(idx / (size_t)limit), col = (int)(idx % (size_t)limit);
    // slices are summed in order; loads go out eight at a time
    const float *p = ws + (size_t)row * n + col;
    const size_t slice = (size_t)mp * n;
    float acc = 0.0f;
    for (int s0 = 0; s0 < splits; s0 += 8) {
      float v8[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) v8[t] = p[(size_t)min(s0 + t, splits - 1) * slice];
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (s0 + t < splits) acc += v8[t];
    }
    const float v = (float)(_Float16)acc;
    const float z = bias ? __fadd_rn(v, bias[col]) : v;
    if (mode == 3) {
      y[(size_t)col * m + row] = z;
    } else {
      y[(size_t)row * n + col] = apply_mode(z, mode);
    }
  }
}

// Readout of channel-major split-K slices ([n][mp] each) for mode 3: one
// thread per 4 rows of a column, slices added in order from zero as in
// f16_skinny_epilogue, fp16 readout, bias, then one 16-byte store along M
// (element stores when y + col * m is not 16-byte aligned).
__global__ __launch_bounds__(256) void f16_splitk_readout_cm(float *__restrict__ y, const float *__restrict__ ws,
                                                            const float *__restrict__ bias, int m, int n,
                                                            int channels, int splits, int vec) {
  const int mp = (m + 15) / 16 * 16;
  const int quads = mp / 4;
  const size_t total = (size_t)channels * quads;
  const size_t slice = (size_t)mp * n;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const int col = (int)(u / (size_t)quads), row = 4 * (int)(u % (size_t)quads);
    if (row >= m) continue;
    const float *p = ws + (size_t)col * mp + row;
    hb_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < splits; s0 += 4) {
      hb_f32x4 v4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) v4[t] = *(const hb_f32x4 *)(p + (size_t)min(s0 + t, splits - 1) * slice);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (s0 + t < splits) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] += v4[t][r];
        }
    }
    const float b = bias ? bias[col] : 0.0f;
    hb_f32x4 out;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = (float)(_Float16)acc[r];
      out[r] = bias ? __fadd_rn(v, b) : v;
    }
    float *dst = y + (size_t)col * m + row;
    if (vec) {
      __builtin_nontemporal_store(out, (hb_f32x4 *)dst);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row + r < m) dst[r] = out[r];
    }
  }
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

int compute_units() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      v <= 0)
    v = 256;
  return v;
}

// Columns per workgroup, split count and blocks per split for the few-rows
// path: 64 columns when n allows (each A element is then re-read by a
// quarter as many workgroups), about one workgroup per CU, at least 4
// k-blocks (one per wave) per split.
int skinny_cols(int n) { return n % 64 == 0 ? 64 : 32; }

// k-blocks per wave: two when the k-blocks cover at least one workgroup per
// CU that way, else one.
void skinny_plan(int k, int n, int &splits, int &kpw) {
  const int kblocks = k / 32, groups = n / skinny_cols(n);
  const int per_wg2 = kSkinnyWaves * 2;
  kpw = (long long)groups * ((kblocks + per_wg2 - 1) / per_wg2) >= compute_units() ? 2 : 1;
  const int per_wg = kSkinnyWaves * kpw;
  splits = (kblocks + per_wg - 1) / per_wg;
}

template <int CF, int KPW>
void launch_skinny_k(int rf, dim3 grid, dim3 block, hipStream_t st, float *ws, const float *x, const uint16_t *packed,
                     int m, int k, int n) {
  if (rf <= 1) {
    hipLaunchKernelGGL((f16_skinny_partial<1, CF, KPW>), grid, block, 0, st, ws, x, packed, m, k, n);
  } else if (rf <= 2) {
    hipLaunchKernelGGL((f16_skinny_partial<2, CF, KPW>), grid, block, 0, st, ws, x, packed, m, k, n);
  } else if (rf <= 4) {
    hipLaunchKernelGGL((f16_skinny_partial<4, CF, KPW>), grid, block, 0, st, ws, x, packed, m, k, n);
  } else if (rf <= 6) {
    hipLaunchKernelGGL((f16_skinny_partial<6, CF, KPW>), grid, block, 0, st, ws, x, packed, m, k, n);
  } else {
    hipLaunchKernelGGL((f16_skinny_partial<8, CF, KPW>), grid, block, 0, st, ws, x, packed, m, k, n);
  }
}

template <int CF>
void launch_skinny(int rf, int kpw, dim3 grid, dim3 block, hipStream_t st, float *ws, const float *x,
                   const uint16_t *packed, int m, int k, int n) {
  if (kpw == 2) launch_skinny_k<CF, 2>(rf, grid, block, st, ws, x, packed, m, k, n);
  else launch_skinny_k<CF, 1>(rf, grid, block, st, ws, x, packed, m, k, n);
}

template <int CF, int TYPE>
void launch_qk0_skinny(int kpw, dim3 grid, dim3 block, hipStream_t st, float *ws, const float *x,
                       const uint8_t *blocks, int m, int k, int n) {
  if (kpw == 8)
    hipLaunchKernelGGL((qk0_skinny_partial<1, CF, 8, TYPE>), grid, block, 0, st, ws, x, blocks, m, k, n);
  else if (kpw == 4)
    hipLaunchKernelGGL((qk0_skinny_partial<1, CF, 4, TYPE>), grid, block, 0, st, ws, x, blocks, m, k, n);
  else if (kpw == 2)
    hipLaunchKernelGGL((qk0_skinny_partial<1, CF, 2, TYPE>), grid, block, 0, st, ws, x, blocks, m, k, n);
  else
    hipLaunchKernelGGL((qk0_skinny_partial<1, CF, 1, TYPE>), grid, block, 0, st, ws, x, blocks, m, k, n);
}

template <int TYPE>
void launch_qk0_skinny_type(int cols, int kpw, dim3 grid, dim3 block, hipStream_t st, float *ws, const float *x,
                            const uint8_t *blocks, int m, int k, int n) {
  if (cols == 64) launch_qk0_skinny<4, TYPE>(kpw, grid, block, st, ws, x, blocks, m, k, n);
  else launch_qk0_skinny<2, TYPE>(kpw, grid, block, st, ws, x, blocks, m, k, n);
}

// Partial sums of the split-K path: one mp x n f32 slice per split, for
// m <= 128 only (0 otherwise).
size_t split_k_bytes(int m, int k, int n) {
  if (m < 1 || m > 128 || k < 32 || n < 32) return 0;
  // splits <= ceil(kblocks / 4) (one k-block per wave at the least)
  const int max_splits = (k / 32 + kSkinnyWaves - 1) / kSkinnyWaves;
  return (size_t)max_splits * (size_t)((m + 15) / 16 * 16) * (size_t)n * 4u;
}

// The fp16 activation image of the ring path: mp rows x k, 2 bytes each.
size_t a_image_bytes(int m, int k) { return hb_round_up((size_t)((m + 15) / 16 * 16) * (size_t)k * 2u, 256); }

// The ring path pays one extra launch (f16_pack_a); it is used from 4 GFLOP
// of work with at least 64 rows (measured: 77x4096x14336 74 -> 29 us,
// 2048x4096x14336 613 -> 250 us, 4096x1536x6144 212 -> 89 us).
// The ring kernel above 128 rows at any size: against the tiled kernels it
// measured equal or faster everywhere (256x1536x4608 30.4 -> 15.1 us,
// 512x1536x1536 30.7 -> 14.9 us, 256x768x3072 14.4 -> 9.8 us).  From 64 to
// 128 rows only from 4 GFLOP, below which the one-launch small kernel and the
// split-K path keep those shapes.
bool ring_worth_it(int m, int k, int n) { return m >= 64 && (m > 128 || 2.0 * m * (double)n * k >= 4e9); }

// Ring tile shapes, cheapest (rounds of resident workgroups) x (work per
// round per CU) / measured efficiency; 128x192 only when n allows.
struct RingShape {
  int bm, bn, occ, eff;
};
constexpr RingShape kRingShapes[] = {{128, 192, 2, 100}, {128, 128, 2, 92}, {64, 64, 4, 60}};

int pick_ring_shape(int m, int n, long long *cost_out = nullptr) {
  const int cus = compute_units();
  int best = -1;
  long long best_cost = -1;
  for (int i = 0; i < 3; ++i) {
    const RingShape t = kRingShapes[i];
    if (n % t.bn != 0 && t.bn == 192) continue;
    const long long tiles = (long long)((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
    const long long slots = (long long)cus * t.occ;
    const long long cost = (tiles + slots - 1) / slots * t.bm * t.bn * t.occ * 100 / t.eff;
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = i;
    }
  }
  if (cost_out) *cost_out = best_cost;
  return best;
}

// Workgroups of the ring kernel's launch for the shape pick_ring_shape takes.
long long ring_tiles(int m, int n) {
  const RingShape t = kRingShapes[pick_ring_shape(m, n)];
  return (long long)((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
}

// The streaming kernel (f16_gemm_stream, one persistent workgroup per CU,
// 256 x 128 tiles, 6 stages of 24 KB) where its tiles occupy at least half of
// the CUs and its cost in the ring shapes' model (rounds of tiles x work per
// tile per CU) is lower than the best ring shape's, or equal with whole
// rounds of tiles.  Measured, us, streaming / ring kernel (one box): chosen at
// 2048x4096x14336 253 / 264, 4096x6144x1536 99.6 / 114, 4096x1536x6144
// 88.0 / 90.3 (equal cost, 3 whole rounds); not chosen at 1024x4096x4096
// 51.4 / 59.6 (the model rates the 64x64 ring tiles cheaper), 4096x1536x4608
// 80.9 / 75.6 (equal cost, 2.25 rounds), 2048x4096x6144 111 / 106, 2048x1536x6144 50.9 / 49.0 (one whole
// round of 128 x 192 ring tiles against one and a half of streaming tiles),
// 512x14336x4096 222 / 125 (64 tiles).  One barrier per two k-steps instead
// of one per k-step measured within 3 %; the 256 x 192 form needs more
// registers than three waves per SIMD hold and spilled (3x slower).
// HTP_OPS_AMD_F16_STREAM gives the initial setting of hb_f16_force_stream;
// HTP_OPS_AMD_F16_STAGGER=ticks sets the odd slots' start delay.
constexpr int kF16StreamBM = 256, kF16StreamBN = 128, kF16StreamStages = 6;

bool f16_stream_setting_ok(int v) { return v >= -1 && v <= 1; }

// -1: automatic, 0: off, 1: on wherever it applies.
std::atomic<int> g_f16_stream{-2};

int f16_stream_mode() {
  int mode = g_f16_stream.load(std::memory_order_relaxed);
  if (mode == -2) {
    const char *v = getenv("HTP_OPS_AMD_F16_STREAM");
    mode = (v && *v && f16_stream_setting_ok(atoi(v))) ? atoi(v) : -1;
    int expected = -2;
    if (!g_f16_stream.compare_exchange_strong(expected, mode)) mode = expected;
  }
  return mode;
}

int f16_stream_stagger(int tiles, int grid) {
  const char *env = getenv("HTP_OPS_AMD_F16_STAGGER");
  if (env && *env && atoi(env) >= 0) return atoi(env);
  const int rounds = tiles % grid == 0 ? tiles / grid : 0;
  return rounds >= 2 ? 500 : 0;
}

bool f16_stream_applies(int m, int k, int n) {
  const int smode = f16_stream_mode();
  if (smode == 0 || k / 32 < kF16StreamStages - 1) return false;
  const int mp = (m + 15) / 16 * 16;
  if ((size_t)mp * (size_t)k * 2u >= ((size_t)1 << 32) || (size_t)n * (size_t)k * 2u >= ((size_t)1 << 32) ||
      (size_t)kF16StreamBM * (size_t)n * 4u >= ((size_t)1 << 32))
    return false;
  if (smode == 1) return true;
  const long long cus = compute_units();
  const long long tiles =
      (long long)((m + kF16StreamBM - 1) / kF16StreamBM) * ((n + kF16StreamBN - 1) / kF16StreamBN);
  long long ring_cost = 0;
  pick_ring_shape(m, n, &ring_cost);
  const long long cost = (tiles + cus - 1) / cus * kF16StreamBM * kF16StreamBN;
  return 2 * tiles >= cus && (cost < ring_cost || (cost == ring_cost && tiles % cus == 0));
}

template <int BM, int BN, int S>
int launch_f16_stream_t(float *y, const int8_t *a, const int8_t *w, const float *bias, int m, int k, int n, int mode,
                        hipStream_t st) {
  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int grid = std::min(compute_units(), (tiles + 7) / 8 * 8) / 8 * 8;
  if (grid < 8) return hb_invalid("f16_gemm_stream grid");
  const int stagger = f16_stream_stagger(tiles, grid);
  if (mode == 1)
    hipLaunchKernelGGL((f16_gemm_stream<BM, BN, 4, 2, 4, S, 1>), dim3(grid), dim3(768), 0, st, y, a, w, bias, m, k, n,
                       tiles_m, tiles_n, stagger);
  else if (mode == 2)
    hipLaunchKernelGGL((f16_gemm_stream<BM, BN, 4, 2, 4, S, 2>), dim3(grid), dim3(768), 0, st, y, a, w, bias, m, k, n,
                       tiles_m, tiles_n, stagger);
  else
    hipLaunchKernelGGL((f16_gemm_stream<BM, BN, 4, 2, 4, S, 0>), dim3(grid), dim3(768), 0, st, y, a, w, bias, m, k, n,
                       tiles_m, tiles_n, stagger);
  return hb_check_launch("f16_gemm_stream");
}

// Narrow streaming tiles for few rows: 128 x 64 (12 stages of 12 KB) and
// 256 x 64 (7 stages of 20 KB).  HTP_OPS_AMD_F16_STREAM_SHAPE=2 / 3 selects
// them wherever the ring path runs (measurement hook); the 256 x 64 form
// also runs by itself at one 256-row tile (below).
int f16_stream_narrow() {
  static const int v = getenv("HTP_OPS_AMD_F16_STREAM_SHAPE") ? atoi(getenv("HTP_OPS_AMD_F16_STREAM_SHAPE")) : 0;
  return v;
}

int launch_f16_stream(float *y, const int8_t *a, const int8_t *w, const float *bias, int m, int k, int n, int mode,
                      hipStream_t st) {
  return launch_f16_stream_t<kF16StreamBM, kF16StreamBN, kF16StreamStages>(y, a, w, bias, m, k, n, mode, st);
}

int launch_ring(float *y, const float *x, const uint16_t *packed, const float *bias, int m, int k, int n, int channels,
                int mode, void *ws, hipStream_t st) {
  const int mp = (m + 15) / 16 * 16;
  const size_t slots = (size_t)mp * k / 8u;
  const int pg = (int)((slots + 255) / 256 < 65536 ? (slots + 255) / 256 : 65536);
  hipLaunchKernelGGL(f16_pack_a, dim3(pg), dim3(256), 0, st, (uint4 *)ws, x, m, k, mp);
  int rc = hb_check_launch("f16_pack_a");
  if (rc) return rc;
  // One 256-row tile (193-256 rows): 256 x 64 streaming tiles read the
  // weights once where they cover half of the CUs (256x4096x14336 70.0 ->
  // 56.4 us, 256x4096x10240 39.5 -> 37.6; at 192 rows the ring kernel stays
  // ahead: 192x4096x10240 31.4 against 35.3).
  // The streaming kernels write row-major rows only; mode 3 takes the ring kernel.
  const bool rows_out = mode != 3;
  const bool narrow_auto = f16_stream_narrow() == 0 && m > 192 && m <= 256 && 2 * ((n + 63) / 64) >= compute_units();
  if (rows_out && f16_stream_mode() != 0 && (f16_stream_narrow() == 2 || narrow_auto) && k / 32 >= 6)
    return launch_f16_stream_t<256, 64, 7>(y, (const int8_t *)ws, (const int8_t *)packed, bias, m, k, n, mode, st);
  if (rows_out && f16_stream_mode() != 0 && f16_stream_narrow() == 3 && k / 32 >= 11)
    return launch_f16_stream_t<128, 64, 12>(y, (const int8_t *)ws, (const int8_t *)packed, bias, m, k, n, mode, st);
  if (rows_out && f16_stream_applies(m, k, n))
    return launch_f16_stream(y, (const int8_t *)ws, (const int8_t *)packed, bias, m, k, n, mode, st);
  const int shape = pick_ring_shape(m, n);
  const RingShape t = kRingShapes[shape];
  const int grid = ((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn);
  const int8_t *a = (const int8_t *)ws, *w = (const int8_t *)packed;
  switch (shape) {
    case 0:
      hipLaunchKernelGGL((f16_gemm_ring<128, 192, 2, 2, 4>), dim3(grid), dim3(256), 0, st, y, a, w, bias, m, k, n,
                         channels, mode);
      break;
    case 1:
      hipLaunchKernelGGL((f16_gemm_ring<128, 128, 2, 2, 4>), dim3(grid), dim3(256), 0, st, y, a, w, bias, m, k, n,
                         channels, mode);
      break;
    default:
      hipLaunchKernelGGL((f16_gemm_ring<64, 64, 2, 2, 4>), dim3(grid), dim3(256), 0, st, y, a, w, bias, m, k, n,
                         channels, mode);
      break;
  }
  return hb_check_launch("f16_gemm_ring");
}

// Split-K ring path for m <= 256: fp16 activation image, f16_ring_splitk on
// 128 x 128 tiles with K split so that the launch has about two workgroups
// per CU (at most kMaxRingSplits slices), then f16_skinny_epilogue.  It
// replaces the few-rows split-K kernel from 33 rows on, whose every column
// group re-reads the fp32 rows (measured, us, few-rows / this path:
// 77x10240x4096 60.7 / 25.0, 128x10240x4096 120 / 31, 77x4096x4096 25.4 /
// 16.6, 64x4096x4096 19.3 / 16.0, 48x2048x8192 20.4 / 17.0, 77x1280x5120
// 17.1 / 14.3; at 32 rows and fewer the few-rows kernel stays ahead:
// 32x4096x4096 13.3 / 14.4, 20x1536x6144 9.5 / 12.5, 1x4096x14336 25.6 /
// 32.7).  Where the ring or the one-launch kernel applies they stay ahead
// too (77x4096x14336 38.7 / 44.2, 77x768x3072 6.7 / 11.1).  Up to 256 rows
// (two row tiles) it replaces the ring kernel where that has no more tiles
// than CUs: 256x10240x4096 68.3 -> 50.8 us, 160x3072x3072 21.7 -> 18.1
// (256x4096x4096 27.7 -> 28.4).
constexpr int kMaxRingSplits = 8;

int ring_splits(int m, int k, int n) {
  const long long tiles = (long long)((m + 127) / 128) * ((n + 127) / 128);
  const long long want = (2LL * compute_units() + tiles - 1) / tiles;
  const int kblocks = k / 32;
  int splits = (int)std::min<long long>(std::min<long long>(want, kMaxRingSplits), kblocks);
  return splits < 1 ? 1 : splits;
}

// 257 to kRingSplitRows rows and k >= 2048: the split-K ring path where
// 128 x 128 tiles fill at most half of the CUs (the few-tile, long-k
// products of im2col convolutions).  Measured, us, ring kernel -> split-K,
// mode 0: 512x11520x1280 71.3 -> 43.5, 1024x11520x1280 84.5 -> 73.5,
// 1024x4608x512 34.8 -> 25.2, 1024x5760x640 41.3 -> 31.5, 512x5760x1280
// 38.0 -> 28.3, 2048x4608x512 39.9 -> 38.2, 1024x2880x640 23.4 -> 23.0; at
// 160 tiles (2048x11520x1280) 122.5 against 120.3.
constexpr int kRingSplitRows = 2048;

bool wide_splitk_shape(int m, int k, int n) {
  const long long tiles128 = ((m + 127) / 128) * (long long)((n + 127) / 128);
  return m > 256 && m <= kRingSplitRows && k >= 2048 && 2 * tiles128 <= compute_units();
}

// Workspace of the split-K ring path: the fp16 image and the slices; 0 where
// the path does not run (more than 256 rows outside wide_splitk_shape).
size_t ring_splitk_bytes(int m, int k, int n) {
  if (m < 1 || k < 32 || n < 32 || (m > 256 && !wide_splitk_shape(m, k, n))) return 0;
  const int slices = m <= 256 ? kMaxRingSplits : ring_splits(m, k, n);
  return a_image_bytes(m, k) + (size_t)slices * (size_t)((m + 15) / 16 * 16) * (size_t)n * 4u;
}

int launch_ring_splitk(float *y, const float *x, const uint16_t *packed, const float *bias, int m, int k, int n,
                       int channels, int mode, void *ws, hipStream_t st) {
  const int mp = (m + 15) / 16 * 16;
  const size_t slots = (size_t)mp * k / 8u;
  const int pg = (int)((slots + 255) / 256 < 65536 ? (slots + 255) / 256 : 65536);
  hipLaunchKernelGGL(f16_pack_a, dim3(pg), dim3(256), 0, st, (uint4 *)ws, x, m, k, mp);
  int rc = hb_check_launch("f16_pack_a");
  if (rc) return rc;
  const int splits = ring_splits(m, k, n);
  const int kps = (k / 32 + splits - 1) / splits;
  const int used = (k / 32 + kps - 1) / kps;  // slices that hold k-steps
  float *part = (float *)((uint8_t *)ws + a_image_bytes(m, k));
  const int tiles = ((m + 127) / 128) * ((n + 127) / 128);
  const int cm = mode == 3;
  hipLaunchKernelGGL((f16_ring_splitk<128, 128, 2, 2, 4>), dim3(tiles, used), dim3(256), 0, st, part,
                     (const int8_t *)ws, (const int8_t *)packed, m, k, n, kps, cm);
  rc = hb_check_launch("f16_ring_splitk");
  if (rc) return rc;
  if (cm) {
    const size_t quads = (size_t)channels * (size_t)(mp / 4);
    const int eg = (int)((quads + 255) / 256 < 4096 ? (quads + 255) / 256 : 4096);
    const int vec = (m % 4 == 0) && aligned(y, 16);
    hipLaunchKernelGGL(f16_splitk_readout_cm, dim3(eg), dim3(256), 0, st, y, part, bias, m, n, channels, used, vec);
    return hb_check_launch("f16_splitk_readout_cm");
  }
  const size_t outs = (size_t)m * (size_t)(mode == 3 ? channels : n);
  const int eg = (int)((outs + 255) / 256 < 4096 ? (outs + 255) / 256 : 4096);
  hipLaunchKernelGGL(f16_skinny_epilogue, dim3(eg), dim3(256), 0, st, y, part, bias, m, n, channels, mode, used);
  return hb_check_launch("f16_skinny_epilogue");
}

// -1 (default): the split-K ring path by the rules of hb_f16_gemm_ws; 0:
// never; 1: for every m <= 256 with a workspace, and from 257 rows where the
// automatic choice takes it (hb_f16_force_splitk; HTP_OPS_AMD_F16_SPLITK
// gives the initial value).
std::atomic<int> g_f16_splitk{-2};

int ring_splitk_mode() {
  int mode = g_f16_splitk.load(std::memory_order_relaxed);
  if (mode == -2) {
    const char *v = getenv("HTP_OPS_AMD_F16_SPLITK");
    mode = (v && *v && f16_stream_setting_ok(atoi(v))) ? atoi(v) : -1;
    int expected = -2;
    if (!g_f16_splitk.compare_exchange_strong(expected, mode)) mode = expected;
  }
  return mode;
}

// Few rows in one launch (f16_small): m <= 128, k <= 3072, a weight image
// of at most 32 MB, and below the ring path's size.  Column fragments per
// workgroup: 4 when that still gives a workgroup per two CUs (and k <= 2048,
// for registers), else 2 when that gives one per CU, else 1.  Returns 0 when
// the shape does not qualify.  hb_f16_gemm_ws and hb_qk0_gemm_ws plan with
// the same function, so they take the same summation order.
int small_cf(int m, int k, int n) {
  if (m > 128 || k > 96 * 32 || (size_t)n * (size_t)k * 2u > ((size_t)32 << 20) || ring_worth_it(m, k, n)) return 0;
  const long long rt = (m + 15) / 16;
  const int cus = compute_units();
  if (n % 64 == 0 && k <= 64 * 32 && rt * (n / 64) >= cus / 2) return 4;
  if (rt * (n / 32) >= cus) return 2;
  return 1;
}

template <int CF, int TYPE>
void launch_small_cf(float *y, const float *x, const void *weights, const float *bias, int m, int k, int n,
                     int channels, int mode, hipStream_t st) {
  const int kblocks = k / 32;
  const dim3 grid((m + 15) / 16, n / (16 * CF)), block(1024);
  if (kblocks <= 16)
    hipLaunchKernelGGL((f16_small<CF, 16, 1, TYPE>), grid, block, 0, st, y, x, weights, bias, m, k, n, channels, mode);
  else if (kblocks <= 32)
    hipLaunchKernelGGL((f16_small<CF, 16, 2, TYPE>), grid, block, 0, st, y, x, weights, bias, m, k, n, channels, mode);
  else if (kblocks <= 64)
    hipLaunchKernelGGL((f16_small<CF, 16, 4, TYPE>), grid, block, 0, st, y, x, weights, bias, m, k, n, channels, mode);
  else if constexpr (CF < 4)
    hipLaunchKernelGGL((f16_small<CF, 16, 6, TYPE>), grid, block, 0, st, y, x, weights, bias, m, k, n, channels, mode);
}

template <int TYPE>
int launch_small(int cf, float *y, const float *x, const void *weights, const float *bias, int m, int k, int n,
                 int channels, int mode, hipStream_t st) {
  if (cf == 4) launch_small_cf<4, TYPE>(y, x, weights, bias, m, k, n, channels, mode, st);
  else if (cf == 2) launch_small_cf<2, TYPE>(y, x, weights, bias, m, k, n, channels, mode, st);
  else launch_small_cf<1, TYPE>(y, x, weights, bias, m, k, n, channels, mode, st);
  return hb_check_launch("f16_small");
}

// -1: automatic, 0: off, 1: on wherever its alignment holds; the initial
// value comes from HTP_OPS_AMD_F16_XSTREAM (hb_f16_force_xstream sets it).
std::atomic<int> g_f16_xstream{-2};

int xstream_mode() {
  int mode = g_f16_xstream.load(std::memory_order_relaxed);
  if (mode == -2) {
    const char *v = getenv("HTP_OPS_AMD_F16_XSTREAM");
    mode = (v && *v && f16_stream_setting_ok(atoi(v))) ? atoi(v) : -1;
    int expected = -2;
    if (!g_f16_xstream.compare_exchange_strong(expected, mode)) mode = expected;
  }
  return mode;
}

template <int BN, int WAVES, int DA, int DB, bool SWAP>
void launch_xstream_form(float *y, const float *x, const uint16_t *packed, const float *bias, int m, int k, int n,
                         int channels, int mode, hipStream_t st) {
  const int grid = ((m + 16 * WAVES - 1) / (16 * WAVES)) * ((n + BN - 1) / BN);
  hipLaunchKernelGGL((f16_gemm_xstream<BN, WAVES, DA, DB, SWAP>), dim3(grid), dim3(64 * WAVES), 0, st, y, x,
                     (const int8_t *)packed, bias, m, k, n, channels, mode);
}

// 8 waves (128 rows) per workgroup sharing one weight ring where their
// workgroups still cover the CUs: 16384x4608x512 155 -> 122 us, 65536x2304x256
// 184 -> 149, 262144x1152x128 291 -> 257 (mode 3); fewer rows keep 4-wave
// workgroups, twice as many (16384x2304x256: 48 against 61.5 us).  A weight
// ring one stage deeper (4 k-steps ahead) or activations 6 k-steps ahead
// measured the same.
template <int BN, bool SWAP>
void launch_xstream_t(float *y, const float *x, const uint16_t *packed, const float *bias, int m, int k, int n,
                      int channels, int mode, hipStream_t st) {
  const long long blocks128 = (long long)((m + 127) / 128) * ((n + BN - 1) / BN);
  if (blocks128 >= compute_units())
    launch_xstream_form<BN, 8, 4, 3, SWAP>(y, x, packed, bias, m, k, n, channels, mode, st);
  else
    launch_xstream_form<BN, 4, 4, 2, SWAP>(y, x, packed, bias, m, k, n, channels, mode, st);
}

// Column chunk of the activation-streaming kernel: 128 or 256 columns.
int xstream_bn(int n) { return n <= 128 ? 128 : 256; }

bool xstream_aligned(const float *y, const float *x, int mode) {
  return aligned(x, 16) && (mode == 3 || aligned(y, 16));
}

// Automatic use: many rows and few columns, where reading the fp32 rows once
// beats converting them to an fp16 image first (the ring path: 8 bytes per
// value moved before the GEMM reads 2 more).  Below a few thousand rows the
// kernel's k loop is latency-bound (its time is flat in m) and the ring
// kernel, which writes every mode, stays ahead.  Measured, us, ring kernel /
// this kernel (the same in modes 0 and 3): 16384x2304x256 74 / 49,
// 65536x2304x256 267 / 145, 16384x4608x512 153 / 120, 8192x4608x512 99.6 /
// 80.0, 8192x2304x256 41.3 / 40.4, 8192x1152x128 21.8 / 16.0, 4096x1152x128
// 16.2 / 15.8; the ring kernel ahead at 4096x2304x256 28.5 / 40.4,
// 4096x4608x512 55.3 / 72.5, 2048x2304x256 23.3 / 40.4.
bool xstream_applies(int m, int n) {
  if (n > 512) return false;
  return m >= (n <= 128 ? 4096 : 8192);
}

int launch_xstream(float *y, const float *x, const uint16_t *packed, const float *bias, int m, int k, int n,
                   int channels, int mode, hipStream_t st) {
  const int bn = xstream_bn(n);
  if (mode == 3) {
    if (bn == 128) launch_xstream_t<128, false>(y, x, packed, bias, m, k, n, channels, mode, st);
    else launch_xstream_t<256, false>(y, x, packed, bias, m, k, n, channels, mode, st);
  } else {
    if (bn == 128) launch_xstream_t<128, true>(y, x, packed, bias, m, k, n, channels, mode, st);
    else launch_xstream_t<256, true>(y, x, packed, bias, m, k, n, channels, mode, st);
  }
  return hb_check_launch("f16_gemm_xstream");
}

}  // namespace

extern "C" {

size_t hb_f16_packed_bytes(int k, int n) {
  if (k <= 0 || n <= 0) return 0;
  return (size_t)k * (size_t)n * 2u;
}

int hb_f16_prepack(uint16_t *d_packed, const uint16_t *d_permuted, int k, int n, hb_stream s) {
  if (!d_packed || !d_permuted) return hb_invalid("hb_f16_prepack null pointer");
  if (k < 32 || k % 32 || n < 32 || n % 32) return hb_invalid("hb_f16_prepack shape");
  if (!aligned(d_permuted, 4) || !aligned(d_packed, 16)) return hb_invalid("hb_f16_prepack alignment");
  const size_t slots = (size_t)n * k / 8u;
  const int grid = (int)((slots + 255) / 256 < 65536 ? (slots + 255) / 256 : 65536);
  hipLaunchKernelGGL(f16_prepack, dim3(grid), dim3(256), 0, hb_resolve_stream(s), (uint4 *)d_packed, d_permuted, k,
                     n);
  return hb_check_launch("f16_prepack");
}

size_t hb_qk0_block_bytes(int type) {
  switch (type) {
    case HB_GGML_Q4_0:
    case HB_GGML_IQ4_NL: return 16u + 128u;
    case HB_GGML_Q8_0: return 16u + 256u;
    default: return 0u;
  }
}

size_t hb_qk0_weight_bytes(int k, int n, int type) {
  if (k <= 0 || n <= 0 || k % 32 || n % 32) return 0;
  return (size_t)k * (size_t)n / 256u * hb_qk0_block_bytes(type);
}

int hb_qk0_prepack(uint16_t *d_packed, const uint8_t *d_blocks, int k, int n, int type, hb_stream s) {
  if (!d_packed || !d_blocks) return hb_invalid("hb_qk0_prepack null pointer");
  if (k < 32 || k % 32 || n < 32 || n % 32) return hb_invalid("hb_qk0_prepack shape");
  const size_t bb = hb_qk0_block_bytes(type);
  if (!bb) return hb_invalid("hb_qk0_prepack type");
  if (!aligned(d_packed, 16)) return hb_invalid("hb_qk0_prepack alignment");
  const size_t slots = (size_t)n * k / 8u;
  const int grid = (int)((slots + 255) / 256 < 65536 ? (slots + 255) / 256 : 65536);
  hipLaunchKernelGGL(qk0_prepack, dim3(grid), dim3(256), 0, hb_resolve_stream(s), (uint4 *)d_packed, d_blocks, k, n,
                     type, (int)bb);
  return hb_check_launch("qk0_prepack");
}

int hb_qk0_gemm_ws(float *d_y, const float *d_x, const uint8_t *d_blocks, int m, int k, int n, int type,
                   void *d_workspace, size_t workspace_bytes, hb_stream s) {
  if (!d_y || !d_x || !d_blocks || !d_workspace) return hb_invalid("hb_qk0_gemm_ws null pointer");
  if (m < 1 || m > 16 || k < 32 || k % 32 || n < 32 || n % 32) return hb_invalid("hb_qk0_gemm_ws shape");
  if (!hb_qk0_block_bytes(type)) return hb_invalid("hb_qk0_gemm_ws type");
  if (workspace_bytes < split_k_bytes(m, k, n)) return hb_invalid("hb_qk0_gemm_ws workspace too small");
  if (!aligned(d_x, 16) || !aligned(d_blocks, 16) || !aligned(d_y, 4) || !aligned(d_workspace, 16))
    return hb_invalid("hb_qk0_gemm_ws alignment");
  hipStream_t st = hb_resolve_stream(s);
  // One row: the whole-K kernel (measured at k=4096, n=14336, m=1: Q4_0 11.0
  // against 14.1 us split-K; Q8_0 25.3 either way, 16 waves keep its
  // registers at one round).
  // One row through the LDS ring (k <= 4096); 2-16 rows on the same plan.
  // HTP_OPS_AMD_QK0_RING (comparisons only): bit 0 off keeps the one-row
  // register-load kernel below, bit 1 off the split-K path for 2-16 rows.
  static const int ring_on = getenv("HTP_OPS_AMD_QK0_RING") ? atoi(getenv("HTP_OPS_AMD_QK0_RING")) : 3;
  if ((ring_on & 2) && m >= 2 && k <= 16 * 8 * 32 && n % 64 == 0) {
    if (type == HB_GGML_Q4_0)
      hipLaunchKernelGGL((qk0_rows_ring<HB_GGML_Q4_0, 16, 8>), dim3(n / 64), dim3(1024), 0, st, d_y, d_x, d_blocks,
                         m, k, n);
    else if (type == HB_GGML_IQ4_NL)
      hipLaunchKernelGGL((qk0_rows_ring<HB_GGML_IQ4_NL, 16, 8>), dim3(n / 64), dim3(1024), 0, st, d_y, d_x,
                         d_blocks, m, k, n);
    else
      hipLaunchKernelGGL((qk0_rows_ring<HB_GGML_Q8_0, 16, 8>), dim3(n / 64), dim3(1024), 0, st, d_y, d_x, d_blocks,
                         m, k, n);
    return hb_check_launch("qk0_rows_ring");
  }
  if ((ring_on & 1) && m == 1 && k <= 16 * 8 * 32) {
    if (type == HB_GGML_Q4_0)
      hipLaunchKernelGGL((qk0_decode_ring<HB_GGML_Q4_0, 16, 8>), dim3(n / 32), dim3(1024), 0, st, d_y, d_x, d_blocks,
                         k, n);
    else if (type == HB_GGML_IQ4_NL)
      hipLaunchKernelGGL((qk0_decode_ring<HB_GGML_IQ4_NL, 16, 8>), dim3(n / 32), dim3(1024), 0, st, d_y, d_x,
                         d_blocks, k, n);
    else
      hipLaunchKernelGGL((qk0_decode_ring<HB_GGML_Q8_0, 16, 8>), dim3(n / 32), dim3(1024), 0, st, d_y, d_x,
                         d_blocks, k, n);
    return hb_check_launch("qk0_decode_ring");
  }
  if (m == 1 && k <= 8 * 16 * 32) {
    if (type == HB_GGML_Q4_0)
      hipLaunchKernelGGL((qk0_decode<HB_GGML_Q4_0, 8, 16, 2>), dim3(n / 32), dim3(512), 0, st, d_y, d_x, d_blocks, k,
                         n);
    else if (type == HB_GGML_IQ4_NL)
      hipLaunchKernelGGL((qk0_decode<HB_GGML_IQ4_NL, 8, 16, 2>), dim3(n / 32), dim3(512), 0, st, d_y, d_x, d_blocks,
                         k, n);
    else
      hipLaunchKernelGGL((qk0_decode<HB_GGML_Q8_0, 16, 8, 2>), dim3(n / 32), dim3(1024), 0, st, d_y, d_x, d_blocks,
                         k, n);
    return hb_check_launch("qk0_decode");
  }
  // Small shapes in one launch, planned as hb_f16_gemm_ws plans them.
  if (const int cf = aligned(d_y, 16) ? small_cf(m, k, n) : 0) {
    if (type == HB_GGML_Q4_0)
      return launch_small<HB_GGML_Q4_0>(cf, d_y, d_x, d_blocks, nullptr, m, k, n, n, 0, st);
    if (type == HB_GGML_IQ4_NL)
      return launch_small<HB_GGML_IQ4_NL>(cf, d_y, d_x, d_blocks, nullptr, m, k, n, n, 0, st);
    return launch_small<HB_GGML_Q8_0>(cf, d_y, d_x, d_blocks, nullptr, m, k, n, n, 0, st);
  }
  int splits = 1, kpw = 1;
  skinny_plan(k, n, splits, kpw);
  const int cols = skinny_cols(n);
  const dim3 grid(n / cols, splits), block(64 * kSkinnyWaves);
  float *ws = (float *)d_workspace;
  if (type == HB_GGML_Q4_0)
    launch_qk0_skinny_type<HB_GGML_Q4_0>(cols, kpw, grid, block, st, ws, d_x, d_blocks, m, k, n);
  else if (type == HB_GGML_Q8_0)
    launch_qk0_skinny_type<HB_GGML_Q8_0>(cols, kpw, grid, block, st, ws, d_x, d_blocks, m, k, n);
  else
    launch_qk0_skinny_type<HB_GGML_IQ4_NL>(cols, kpw, grid, block, st, ws, d_x, d_blocks, m, k, n);
  int rc = hb_check_launch("qk0_skinny_partial");
  if (rc) return rc;
  const size_t outs = (size_t)m * (size_t)n;
  const int eg = (int)((outs + 255) / 256 < 4096 ? (outs + 255) / 256 : 4096);
  hipLaunchKernelGGL(f16_skinny_epilogue, dim3(eg), dim3(256), 0, st, d_y, ws, (const float *)nullptr, m, n, n, 0,
                     splits);
  return hb_check_launch("f16_skinny_epilogue");
}

size_t hb_f16_workspace_bytes(int m, int k, int n) {
  if (m < 1 || k < 32 || n < 32) return 0;
  const size_t ring = ring_worth_it(m, k, n) ? a_image_bytes(m, k) : 0;
  const size_t partials = split_k_bytes(m, k, n);
  const size_t ring_partials = ring_splitk_bytes(m, k, n);
  return std::max(std::max(ring, partials), ring_partials);
}

int hb_f16_gemm_ws(float *d_y, const float *d_x, const uint16_t *d_packed, const float *d_bias, int m, int k, int n,
                   int channels, int mode, void *d_workspace, size_t workspace_bytes, hb_stream s) {
  if (!d_y || !d_x || !d_packed) return hb_invalid("hb_f16_gemm null pointer");
  if (m < 1 || k < 32 || k % 32 || n < 32 || n % 32 || channels < 1 || channels > n || mode < 0 || mode > 3 ||
      (mode != 3 && channels != n))
    return hb_invalid("hb_f16_gemm shape/mode");
  if (!aligned(d_x, 16) || !aligned(d_packed, 16) || !aligned(d_y, 4) || (d_bias && !aligned(d_bias, 4)))
    return hb_invalid("hb_f16_gemm alignment");
  hipStream_t st = hb_resolve_stream(s);
  const int xs = xstream_mode();
  if (xs != 0 && xstream_aligned(d_y, d_x, mode) && (xs == 1 || xstream_applies(m, n)))
    return launch_xstream(d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, st);
  const size_t splitk_need = ring_splitk_bytes(m, k, n);
  const bool splitk_ok = ring_splitk_mode() != 0 && splitk_need && d_workspace && workspace_bytes >= splitk_need &&
                         aligned(d_workspace, 256);
  if (splitk_ok && ring_splitk_mode() == 1)
    return launch_ring_splitk(d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, d_workspace, st);
  // Tiled variant by output size; the split-K paths take over when that grid
  // has no more workgroups than CUs, and for m <= 16, where a tile's rows are
  // mostly padding (measured at k=4096, n=14336: m=1 65 -> 28 us;
  // 77x14336x4096: 264 -> 80 us; 64x4096x4096, 256 tiles of 32x32: 40.6 ->
  // 19.7 us).
  const long long big = ((m + 127) / 128) * (long long)((n + 127) / 128);
  const long long mid = ((m + 63) / 64) * (long long)((n + 63) / 64);
  const long long small = ((m + 31) / 32) * (long long)((n + 31) / 32);
  const long long tiled_wgs = big >= 256 ? big : mid >= 128 ? mid : small;
  // From 33 rows the split-K ring path, except where the ring kernel has
  // more tiles than CUs at 4 GFLOP or more (77x4096x14336: 38.4 against
  // 44.2 us; counted in the ring's own tiles: 256x11520x1280, 80 tiles of
  // 64 x 64, 67.7 on the ring against 27.3) and where the one-launch kernel applies to under 12 MB of
  // weights (77x768x3072: 6.7 against 11.1 us, 64x2048x2048 10.4 against
  // 11.3).  Measured, us, previous choice / split-K ring: 100x3072x3072 28.6
  // / 14.4 and 128x3072x3072 28.8 / 15.1 (one launch), 48x2048x8192 20.4 /
  // 17.0 and 77x1280x5120 17.1 / 14.3 (one launch, 13-34 MB of weights).
  const bool ring_here = ring_worth_it(m, k, n) && tiled_wgs > compute_units() && ring_tiles(m, n) > compute_units();
  const bool splitk_here = splitk_ok && m > 32 && m <= 256 && !ring_here;
  const int cf = aligned(d_y, 16) ? small_cf(m, k, n) : 0;
  if (splitk_here && (!cf || (size_t)n * (size_t)k * 2u >= ((size_t)12 << 20)))
    return launch_ring_splitk(d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, d_workspace, st);
  // From 257 rows: the split-K ring path wherever it has a workspace
  // (wide_splitk_shape).
  if (splitk_ok && m > 256)
    return launch_ring_splitk(d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, d_workspace, st);
  if (cf) return launch_small<0>(cf, d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, st);
  // The split-K path holds m <= 128 rows (8 row fragments) of partial sums.
  const size_t need = split_k_bytes(m, k, n);
  if (m <= 128 && d_workspace && need && workspace_bytes >= need && aligned(d_workspace, 16) &&
      (tiled_wgs <= compute_units() || m <= 16)) {
    int splits = 1, kpw = 1;
    skinny_plan(k, n, splits, kpw);
    const int cols = skinny_cols(n);
    const dim3 grid(n / cols, splits), block(64 * kSkinnyWaves);
    float *ws = (float *)d_workspace;
    const int rf = (m + 15) / 16;
    if (cols == 64) launch_skinny<4>(rf, kpw, grid, block, st, ws, d_x, d_packed, m, k, n);
    else launch_skinny<2>(rf, kpw, grid, block, st, ws, d_x, d_packed, m, k, n);
    int rc = hb_check_launch("f16_skinny_partial");
    if (rc) return rc;
    const size_t outs = (size_t)m * (size_t)(mode == 3 ? channels : n);
    const int eg = (int)((outs + 255) / 256 < 4096 ? (outs + 255) / 256 : 4096);
    hipLaunchKernelGGL(f16_skinny_epilogue, dim3(eg), dim3(256), 0, st, d_y, ws, d_bias, m, n, channels, mode,
                       splits);
    return hb_check_launch("f16_skinny_epilogue");
  }
  if (d_workspace && ring_worth_it(m, k, n) && workspace_bytes >= a_image_bytes(m, k) && aligned(d_workspace, 256) &&
      aligned(d_y, 16))
    return launch_ring(d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, d_workspace, st);
  if (big >= 256) {
    hipLaunchKernelGGL((f16_gemm_tiles<128, 128, 2, 2>), dim3((int)big), dim3(256), 0, st, d_y, d_x, d_packed, d_bias,
                       m, k, n, channels, mode);
  } else if (mid >= 128) {
    hipLaunchKernelGGL((f16_gemm_tiles<64, 64, 2, 2>), dim3((int)mid), dim3(256), 0, st, d_y, d_x, d_packed, d_bias,
                       m, k, n, channels, mode);
  } else {
    hipLaunchKernelGGL((f16_gemm_tiles<32, 32, 2, 2>), dim3((int)small), dim3(256), 0, st, d_y, d_x, d_packed, d_bias,
                       m, k, n, channels, mode);
  }
  return hb_check_launch("f16_gemm_tiles");
}

int hb_f16_force_xstream(int setting) {
  if (!f16_stream_setting_ok(setting)) return hb_invalid("hb_f16_force_xstream setting");
  const int prev = xstream_mode();
  g_f16_xstream.store(setting, std::memory_order_relaxed);
  return prev;
}

int hb_f16_force_splitk(int setting) {
  if (!f16_stream_setting_ok(setting)) return hb_invalid("hb_f16_force_splitk setting");
  const int prev = ring_splitk_mode();
  g_f16_splitk.store(setting, std::memory_order_relaxed);
  return prev;
}

int hb_f16_force_stream(int setting) {
  if (!f16_stream_setting_ok(setting)) return hb_invalid("hb_f16_force_stream setting");
  const int prev = f16_stream_mode();
  g_f16_stream.store(setting, std::memory_order_relaxed);
  return prev;
}

int hb_f16_gemm(float *d_y, const float *d_x, const uint16_t *d_packed, const float *d_bias, int m, int k, int n,
                int channels, int mode, hb_stream s) {
  return hb_f16_gemm_ws(d_y, d_x, d_packed, d_bias, m, k, n, channels, mode, nullptr, 0, s);
}


size_t hb_qkv_gemm_workspace_bytes(int tokens, int input_dim) {
  if (tokens < 1 || input_dim < 32) return 0;
  return a_image_bytes(tokens, input_dim);
}

int hb_qkv_gemm(uint16_t *d_q, uint16_t *d_k, uint16_t *d_v, const float *d_x, const uint16_t *d_packed,
                const float *d_bias, const float *d_q_norm, const float *d_k_norm, const float *d_pe, int rope_offset,
                int rope_count, int tokens, int input_dim, int n_heads, int head_dim, int token_tiles, int out_offset,
                void *d_workspace, size_t workspace_bytes, hb_stream s) {
  if (!d_q || !d_k || !d_v || !d_x || !d_packed || !d_q_norm || !d_k_norm || !d_workspace)
    return hb_invalid("hb_qkv_gemm null pointer");
  if (tokens <= 0 || input_dim < 32 || input_dim % 32 || n_heads <= 0 || (head_dim != 64 && head_dim != 128) ||
      (n_heads * head_dim) % 128 || out_offset < 0 || out_offset % 32 ||
      out_offset / 32 + (tokens + 31) / 32 > token_tiles)
    return hb_invalid("hb_qkv_gemm shape");
  if (workspace_bytes < a_image_bytes(tokens, input_dim)) return hb_invalid("hb_qkv_gemm workspace too small");
  if (!aligned(d_q, 16) || !aligned(d_k, 16) || !aligned(d_v, 16) || !aligned(d_x, 16) || !aligned(d_packed, 16) ||
      !aligned(d_workspace, 256) || (d_bias && !aligned(d_bias, 4)) || (d_pe && !aligned(d_pe, 16)))
    return hb_invalid("hb_qkv_gemm alignment");
  if (d_pe && (rope_offset < 0 || rope_count <= 0)) d_pe = nullptr;  // the reference skips the rotation
  hipStream_t st = hb_resolve_stream(s);
  const int m = tokens, k = input_dim, n = 3 * n_heads * head_dim;
  const int mp = (m + 15) / 16 * 16;
  const size_t slots = (size_t)mp * k / 8u;
  const int pg = (int)((slots + 255) / 256 < 65536 ? (slots + 255) / 256 : 65536);
  hipLaunchKernelGGL(f16_pack_a, dim3(pg), dim3(256), 0, st, (uint4 *)d_workspace, d_x, m, k, mp);
  int rc = hb_check_launch("f16_pack_a");
  if (rc) return rc;
  // 128 x 192 tiles (three heads of 64) where the heads allow, else 128 x 128
  const int bn = head_dim == 64 && (n_heads * head_dim) % 192 == 0 ? 192 : 128;
  const int grid = ((m + 127) / 128) * (n / bn);
  const int8_t *a = (const int8_t *)d_workspace, *w = (const int8_t *)d_packed;
  if (bn == 192)
    hipLaunchKernelGGL((f16_qkv_ring<64, 192>), dim3(grid), dim3(256), 0, st, d_q, d_k, d_v, a, w, d_bias, d_q_norm,
                       d_k_norm, d_pe, rope_offset, rope_count, m, k, n_heads, token_tiles, out_offset / 32);
  else if (head_dim == 64)
    hipLaunchKernelGGL((f16_qkv_ring<64, 128>), dim3(grid), dim3(256), 0, st, d_q, d_k, d_v, a, w, d_bias, d_q_norm,
                       d_k_norm, d_pe, rope_offset, rope_count, m, k, n_heads, token_tiles, out_offset / 32);
  else
    hipLaunchKernelGGL((f16_qkv_ring<128, 128>), dim3(grid), dim3(256), 0, st, d_q, d_k, d_v, a, w, d_bias,
                       d_q_norm, d_k_norm, d_pe, rope_offset, rope_count, m, k, n_heads, token_tiles, out_offset / 32);
  return hb_check_launch("f16_qkv_ring");
}

}  // extern "C"
