/*
 * hb_*: the thin C ABI between the C host library and the gfx950 kernels.
 * Plain pointers, sizes and status codes only.  Every pointer named d_* is a
 * device address; every kernel call is asynchronous on the given stream
 * (NULL = the library's own stream on the current device).
 *
 * This layer replaces the reference's DSP-side kernel entry points:
 *   hb_w8a8_linear / _quantize / _gemm  reference include/dsp/ops.h:20-31,
 *       src/dsp/ops/linear_w8a8.c:327-558 (hmx_mat_mul_native_w8a8*)
 *   hb_w8a8_prepack   consumes the constants blob of reference include/op_reg.h:80-85
 *       (header checks src/dsp/op_executor.cc:331-335); no reference counterpart:
 *       the reference re-copies weights from DDR on every call
 *       (src/dsp/ops/linear_w8a8.c:242-268, :459)
 *   hb_f16_gemm       reference src/dsp/ops/mat_mul.c:937-1049
 *       (hmx_mat_mul_f16_epilogue, hmx_mat_mul_permuted_w16a32)
 *   hb_f16_prepack    no reference counterpart (reference copies the permuted
 *       weight into VTCM per call, src/dsp/ops/mat_mul.c:157-244)
 *   hb_qk0_prepack    replaces the per-call dequantization of Q4_0 / Q8_0 /
 *       IQ4_NL super-blocks (dequantize_permuted_weight_chunk_qk_0_to_fp16_hvx,
 *       src/dsp/ops/mat_mul.c:330-588) feeding hmx_mat_mul_permuted_qk_0_d16a32
 *       (:1601-1720); the GEMM is then hb_f16_gemm
 *
 * Status codes: 0 success, HB_E_INVAL bad argument, HB_E_NODEV no usable GPU,
 * HB_E_HIP a HIP runtime error (text in hb_last_error()), HB_E_NOMEM.
 */
#ifndef HTP_OPS_HB_H
#define HTP_OPS_HB_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HB_OK 0
#define HB_E_HIP (-5)
#define HB_E_NOMEM (-12)
#define HB_E_NODEV (-19)
#define HB_E_INVAL (-22)

typedef void *hb_stream; /* a hipStream_t */
typedef void *hb_event;  /* a hipEvent_t */
typedef void *hb_graph;  /* an instantiated hipGraphExec_t */

/* ---- runtime ------------------------------------------------------------- */
int hb_device_count(void);
int hb_init(int device); /* selects the device for the calling thread and creates the library stream */
const char *hb_last_error(void);
hb_stream hb_default_stream(void);
int hb_malloc(void **d_ptr, size_t bytes);
int hb_free(void *d_ptr);
int hb_host_malloc(void **h_ptr, size_t bytes); /* pinned */
int hb_host_free(void *h_ptr);
int hb_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes, hb_stream s);
int hb_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes, hb_stream s);
int hb_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, hb_stream s);
/* Device -> host copy queued on s without waiting (h_dst pinned, e.g. a
 * host rpcmem buffer); complete once later work on s, or an event recorded
 * after it, has completed. */
int hb_memcpy_d2h_async(void *h_dst, const void *d_src, size_t bytes, hb_stream s);
int hb_memset(void *d_dst, int value, size_t bytes, hb_stream s);
int hb_stream_create(hb_stream *s);
int hb_stream_destroy(hb_stream s);
int hb_stream_sync(hb_stream s);
int hb_device_sync(void);
int hb_event_create(hb_event *e);
int hb_event_destroy(hb_event e);
int hb_event_record(hb_event e, hb_stream s);
int hb_event_sync(hb_event e);
int hb_event_elapsed_ms(float *ms, hb_event start, hb_event stop);
/* Graph capture of the work enqueued on s between begin and end (kernel
 * launches of this library only: no memset or copy is captured by it); the
 * instantiated graph replays that work on any stream. */
int hb_graph_begin(hb_stream s);
int hb_graph_end(hb_graph *g, hb_stream s);
int hb_graph_launch(hb_graph g, hb_stream s);
int hb_graph_destroy(hb_graph g);

/* ---- W8A8 (opcode 15) ----------------------------------------------------- */

/*
 * Packed weight image produced once per constants blob by hb_w8a8_prepack.
 * kp = k rounded up to 64.  Sections (byte offsets from the image base):
 *   [0]                      int8 W in 16(n) x 64(k) MFMA tiles: element (n,k) at
 *                            ((n/16)*(kp/64) + k/64)*1024 + ((n%16) + 16*((k%64)/16))*16 + k%16,
 *                            zero for k >= k_real
 *   [HB_W8A8_SW]             f32 sw[n]        per-column scale (copied from the blob)
 *   [HB_W8A8_DELTA]          i32 delta[n]     128*(sum_k W(n,k) - blob.sums[n]), wrapping
 *   [HB_W8A8_WSUM128]        i32 wsum128[n]   128*sum_k W(n,k), wrapping
 *   [HB_W8A8_INV]            f32 inv[k]       smoothing vector (copied from the blob)
 */
enum { HB_W8A8_WEIGHTS = 0, HB_W8A8_SW = 1, HB_W8A8_DELTA = 2, HB_W8A8_WSUM128 = 3, HB_W8A8_INV = 4 };
size_t hb_w8a8_packed_bytes(int k, int n);
size_t hb_w8a8_packed_offset(int k, int n, int section);

/* Blob (device copy of the constants buffer, header already validated) -> packed image. */
int hb_w8a8_prepack(void *d_packed, const uint8_t *d_blob, int k, int n, hb_stream s);

/* Workspace for quantized activations: int8 q (mp*kp bytes, mp = m rounded up
 * to 16) then f32 scales[mp]. */
size_t hb_w8a8_workspace_bytes(int m, int k);

/*
 * Per-token dynamic quantization (reference linear_w8a8.c:34-120):
 *   t = x*inv; s = max(max|t|/127, 1e-12); u = rint(clamp(t*(1/s)+128, 1, 255))
 * writes q = u - 128 and s (f32[m]).  q uses the weights' tile layout:
 * element (m,k) at ((m/16)*(kp/64) + k/64)*1024 + ((m%16) + 16*((k%64)/16))*16 + k%16,
 * zero for k >= k_real; rows m..mp-1 are left unwritten.
 */
int hb_w8a8_quantize(int8_t *d_q, float *d_scales, const float *d_x, const float *d_inv, int m, int k,
                     hb_stream s);

/* Output epilogues of hb_w8a8_gemm. */
enum {
  HB_W8A8_EPI_SCALE = 0,      /* y = (float)(acc - 128*sums) * sw[n] * s[m], f32 [m][n] */
  HB_W8A8_EPI_SCALE_GELU = 1, /* GELU (tanh form) of the above (no reference opcode) */
  HB_W8A8_EPI_RAW = 2,        /* int32 raw accumulator sum_k u*W, stored as [m][n] int32 */
};

/* INT8 GEMM on quantized activations + fused epilogue; picks the decode
 * (m <= 16) or tiled kernel.  d_y is 16-byte aligned with row stride ldy
 * (elements, >= n, a multiple of 4). */
int hb_w8a8_gemm(void *d_y, int ldy, const int8_t *d_q, const float *d_scales, const void *d_packed, int m, int k,
                 int n, int epilogue, hb_stream s);

/* Tuning and test hook: pins the tiled kernel's shape for every later call
 * (index into 128x192, 256x192, 128x128, 256x256, 64x64, then 5: the
 * persistent streaming kernel with 256x128 tiles, for k >= 320, and 6: the
 * same with 256x192 tiles, for k >= 256, except with the GELU epilogue, which
 * runs shape 5 instead; shapes 192 wide apply only when n % 192 == 0) or
 * restores automatic choice with -1.
 * Returns the previous setting.  Results are identical for every shape.
 * The environment variable HTP_OPS_AMD_W8A8_TILE gives the initial value. */
int hb_w8a8_force_tile(int index);

/* Which kernel hb_w8a8_gemm runs for this shape (after hb_w8a8_force_tile and
 * the environment): HB_W8A8_CHOICE_DECODE (m <= 16, weight-streaming decode
 * kernel), HB_W8A8_CHOICE_DECODE_TILES (17-80 rows over few output tiles: the
 * decode kernel per 16-row tile), or the tile index as hb_w8a8_force_tile
 * numbers them (5 and 6: the persistent streaming kernel with 128- and
 * 192-column tiles; with the GELU epilogue 6 runs as 5); HB_E_INVAL on an
 * invalid shape.  A measurement and test hook; no counterpart in the
 * reference. */
#define HB_W8A8_CHOICE_DECODE (-1)
#define HB_W8A8_CHOICE_DECODE_TILES (-2)
int hb_w8a8_gemm_choice(int m, int k, int n);

/* The output tile of that choice for the scale epilogue: *bm rows by *bn
 * columns per workgroup tile (16 x 16 for the decode kernels).  Returns the
 * choice, or HB_E_INVAL.  Fills opcode 15's profile mode 3. */
int hb_w8a8_gemm_tile(int m, int k, int n, int *bm, int *bn);

/* Workspace that lets hb_w8a8_linear take its split-K path where one applies
 * (33-256 rows with long rows, K from 8192 or from 5120 above 128 rows, whose
 * 128 x 128 output tiles number fewer than half of the CUs: eight int32
 * partial-sum slices of ceil(m/16)*16 x n after the quantized rows and
 * scales); equal to hb_w8a8_workspace_bytes(m, k) where none applies.  The
 * results are the same bits with either workspace.  No counterpart in the
 * reference, whose executor sizes its own scratch (op_executor.cc). */
size_t hb_w8a8_linear_workspace_bytes(int m, int k, int n);

/* Full opcode-15 computation: quantize + GEMM + epilogue (workspace from hb_w8a8_workspace_bytes).
 * With the SCALE or SCALE_GELU epilogue, 16-byte aligned x and y and K a
 * multiple of 32, small problems run as one launch that quantizes its own
 * rows: m == 1 (K <= 16384), 2 <= m <= 4 (K <= 4096), and 5 <= m <= 128 with
 * K <= 1536 and ceil(m/16) * n * K <= 16 MB (HTP_OPS_AMD_W8A8_SMALL=0 turns
 * the last one off).  Every path gives the same bits. */
int hb_w8a8_linear(float *d_y, const float *d_x, const void *d_packed, int m, int k, int n, int epilogue,
                   void *d_workspace, size_t workspace_bytes, hb_stream s);

/* No counterpart in the reference: hb_w8a8_linear for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same computation and bits as
 * hb_w8a8_linear, with its workspace in a library-owned static device array
 * of HB_W8A8_STATIC_SCRATCH_BYTES (32 MiB) per GPU, held until the process
 * ends; hb_w8a8_workspace_bytes(m, k) must not exceed it (e.g. 4096 x 6144
 * fits, 4096 x 8192 does not), else HB_E_INVAL.  The split-K path runs where
 * hb_w8a8_linear_workspace_bytes(m, k, n) fits too.  Allocates nothing: no
 * hipMalloc, no allocating library call.  Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (other streams, other
 * threads) race; calls in one stream are ordered.  hb_init(device) prepares
 * the device's array (hb_w8a8_static_setup); a first call on a device that
 * was not initialised prepares it then. */
#define HB_W8A8_STATIC_SCRATCH_BYTES (32u << 20)
int hb_w8a8_static_setup(int device); /* with `device` current */
int hb_w8a8_linear_noalloc(float *d_y, const float *d_x, const void *d_packed, int m, int k, int n, int epilogue,
                           hb_stream s);

/* CPU-control variant: raw accumulator byte planes in the reference's export
 * format (reference linear_w8a8.c:209-227) written over the f32 output tensor. */
int hb_w8a8_planes_from_raw(uint8_t *d_out, const int32_t *d_raw, int m, int n, hb_stream s);

/* The epilogue of hb_w8a8_gemm as its own launch, for the opcode-15 profile
 * mode 2 split of MAC from readout (reference linear_w8a8.c:488-500): raw
 * holds hb_w8a8_gemm's HB_W8A8_EPI_RAW output (sum_k u*W per element,
 * row stride n), y gets the HB_W8A8_EPI_SCALE / _SCALE_GELU values of the
 * same request, bit for bit (row stride ldy >= n).  n % 16 == 0; y and raw
 * 16-byte aligned, ldy % 4 == 0. */
int hb_w8a8_readout(float *d_y, int ldy, const int32_t *d_raw, const float *d_scales, const void *d_packed, int m,
                    int k, int n, int epilogue, hb_stream s);

/* ---- packed-F16 GEMM (opcodes 1 and 16) ------------------------------------ */

/* Permuted fp16 weight (reference layout) -> 16(n) x 32(k) MFMA tiles:
 * element (n,k) at ((n/16)*(k/32) + k/32)*512 + ((n%16) + 16*((k%32)/8))*8 + k%8 (fp16 units). */
size_t hb_f16_packed_bytes(int k, int n);
int hb_f16_prepack(uint16_t *d_packed, const uint16_t *d_permuted, int k, int n, hb_stream s);

/* Quantized weights of opcodes 2/3/4 (ggml type ids, reference
 * include/dsp/quants.h:33-54): super-blocks of 256 weights, 8 fp16 scales then
 * 128 nibble bytes (Q4_0, IQ4_NL; 144 bytes) or 256 int8 (Q8_0; 272 bytes),
 * covering consecutive positions of the permuted fp16 layout.  hb_qk0_prepack
 * dequantizes them into the hb_f16_prepack image (value * scale rounded once
 * to fp16), so the product then runs through hb_f16_gemm. */
enum { HB_GGML_Q4_0 = 2, HB_GGML_Q8_0 = 8, HB_GGML_IQ4_NL = 20 };
size_t hb_qk0_block_bytes(int type);           /* 0 for an unknown type */
size_t hb_qk0_weight_bytes(int k, int n, int type);
int hb_qk0_prepack(uint16_t *d_packed, const uint8_t *d_blocks, int k, int n, int type, hb_stream s);
/* Few rows (1 <= m <= 16) straight from the super-blocks, each weight fragment
 * dequantized in registers (the same fp16 values as hb_qk0_prepack), mode 0,
 * no bias; workspace of at least hb_f16_workspace_bytes(m, k, n).  m == 1 with
 * k <= 4096 runs one whole-K kernel per 32-column tile (the workspace is not
 * touched); otherwise the split-K path of hb_f16_gemm_ws, equal bit for bit to
 * hb_f16_gemm_ws on the hb_qk0_prepack image.  Replaces the
 * per-call dequantization of hmx_mat_mul_permuted_qk_0_d16a32
 * (reference src/dsp/ops/mat_mul.c:1601-1720) for decode-sized calls. */
int hb_qk0_gemm_ws(float *d_y, const float *d_x, const uint8_t *d_blocks, int m, int k, int n, int type,
                   void *d_workspace, size_t workspace_bytes, hb_stream s);

/*
 * y = epilogue(fp16(fp16(x) @ W)); x f32 [m][k]; bias f32[channels] or NULL.
 * Small shapes (m <= 128, k <= 3072, a weight image of at most 32 MB, a
 * 16-byte aligned y) run as one kernel over the whole K per 16-row tile, with
 * or without a workspace.
 * mode 0: + bias; 1: + bias, GELU (tanh form); 2: + bias, QuickGELU;
 * mode 3: + bias, stored channel-major y[c][m] for c < channels.
 */
int hb_f16_gemm(float *d_y, const float *d_x, const uint16_t *d_packed, const float *d_bias, int m, int k, int n,
                int channels, int mode, hb_stream s);

/* Workspace of hb_f16_gemm_ws: the largest of the few-rows (m <= 128) split-K
 * partial sums, for 64 or more rows and at least 4 GFLOP the fp16 activation
 * image of the ring path (2 * ceil(m/16)*16 * k bytes), and for m <= 128 that
 * image plus eight fp32 partial-sum slices of ceil(m/16)*16 x n for m <= 256
 * (the split-K ring path); 0 when none applies (the tiled kernel needs none). */
size_t hb_f16_workspace_bytes(int m, int k, int n);

/* Tuning and test hook of the F16 path for 64 rows or more with a workspace:
 * -1 restores the automatic choice (the persistent streaming kernel with
 * 256 x 128 tiles where they occupy at least half of the CUs and spread more
 * evenly than the ring kernel's, else the one-tile-per-workgroup ring
 * kernel), 0 keeps the ring
 * kernel, 1 runs the streaming kernel wherever it applies (k >= 160).
 * Returns the previous setting.  Results are identical either way.  The
 * environment variable HTP_OPS_AMD_F16_STREAM gives the initial value. */
int hb_f16_force_stream(int setting);

/* Pins the activation-streaming F16 kernel (f16_gemm_xstream: the fp32
 * activations read once, converted in registers, for many rows and few
 * columns): -1 restores the automatic choice, 0 never, 1 wherever x (and y
 * outside mode 3) are 16-byte aligned.  Returns the previous setting.  The
 * sums are those of the other F16 kernels.  No counterpart in the reference;
 * HTP_OPS_AMD_F16_XSTREAM gives the initial value. */
int hb_f16_force_xstream(int setting);

/* Pins the split-K ring path of hb_f16_gemm_ws (f16_ring_splitk slices added
 * in order by a readout kernel): -1 restores the automatic choice, 0 never
 * (the ring or tiled kernel, whose sums are those of hb_f16_gemm), 1 for
 * every m <= 256 given a large enough workspace (from 257 rows it runs only
 * where the automatic choice takes it).  Returns the previous
 * setting.  Split sums may differ from the unsplit ones in the last fp32 bit
 * before the fp16 readout.  No counterpart in the reference;
 * HTP_OPS_AMD_F16_SPLITK gives the initial value. */
int hb_f16_force_splitk(int setting);

/* hb_f16_gemm with a workspace: for m <= 128, a workspace of at least
 * hb_f16_workspace_bytes, and either m <= 16 or a shape whose output tiles
 * (of the size hb_f16_gemm would use) number no more than the device's CUs, K
 * is split across workgroups and the partial sums are added in a fixed order
 * before the fp16 readout rounding and the epilogue (two kernels; from 33
 * rows on, x is first converted to fp16 MFMA tiles and each split covers all
 * rows of a 128 x 128 tile, so the weights are read once).  The same
 * split-K ring path serves 257 to 2048 rows with k >= 2048 where 128 x 128
 * output tiles would fill at most half of the CUs.
 * Otherwise, with a workspace of at least hb_f16_workspace_bytes, a 16-byte
 * aligned output and 64 or more rows (4 GFLOP or more), x is converted once
 * into fp16 MFMA tiles in the workspace and both operands stream through the
 * direct-to-LDS ring of the int8 GEMM; the result equals hb_f16_gemm bit for
 * bit.  Otherwise identical to hb_f16_gemm. */
int hb_f16_gemm_ws(float *d_y, const float *d_x, const uint16_t *d_packed, const float *d_bias, int m, int k, int n,
                   int channels, int mode, void *d_workspace, size_t workspace_bytes, hb_stream s);

/*
 * Opcode 19 model auxiliary ops on f32 tensors (replaces hvx_model_aux_f32,
 * reference src/dsp/ops/mat_mul.c:2488-2501; argument meaning as in
 * NativeAuxParams, op_reg.h).  d_w / d_b may be NULL where the mode allows.
 *   0 LayerNorm rows of width (+w[i], +b[i]); 1 RMSNorm rows; 9 LayerNorm rows
 *   then v += v*w, v += b (per batch unless other_count == width); 2 GroupNorm
 *   over spatial*channels/groups values with per-channel w/b; for 0/1/2/9 a
 *   nonzero activation applies SiLU;  3/4 x + / * w[i % other_count];
 *   5/6/7 SiLU / GELU-tanh / QuickGELU;  8 transpose [batch][width][spatial]
 *   -> [batch][spatial][width];  10 x*w[batch-or-0][i % width] + b[i];
 *   11 rotary embedding, x [batch][token][head][width], 2x2 matrices w per
 *   (batch-or-0, token, pair), y [batch][head][token][width];  12 SiLU(gate)*up
 *   from rows of `channels` values (activation 0: [up | gate], 1: [gate | up]);
 *   13 as 12, each output row prefixed by `groups` attention values from w.
 * The caller validates shapes as opcode 19 does; this checks only what the
 * kernels index with.
 */
int hb_model_aux(float *d_y, const float *d_x, const float *d_w, const float *d_b, int mode, int count, int width,
                 int channels, int spatial, int groups, int batch, int other_count, int activation, float eps,
                 hb_stream s);

/* Workspace for hb_model_aux_ws: nonzero only for group norms (mode 2) with
 * few long groups, which then split each group over many workgroups (three
 * launches; the statistics are added in a fixed order, so the result does not
 * depend on the split).  The workspace holds no state between calls. */
size_t hb_model_aux_workspace_bytes(int mode, int channels, int spatial, int groups, int batch);
int hb_model_aux_ws(float *d_y, const float *d_x, const float *d_w, const float *d_b, int mode, int count, int width,
                    int channels, int spatial, int groups, int batch, int other_count, int activation, float eps,
                    void *d_workspace, size_t workspace_bytes, hb_stream s);

/*
 * Opcodes 8/10/11/12 post-processing (reference src/dsp/ops/mat_mul.c:1051-1371):
 * d_raw is the packed-F16 GEMM output of one call (tokens x 3*n_heads*head_dim
 * f32, fp16-exact values: hb_f16_gemm mode 0 without bias).  Per head, Q and K
 * get bias, RMS norm with q_norm / k_norm (head_dim values each) and, with
 * d_pe, the rotary 2x2 matrices of token rope_offset + row (head_dim/2
 * matrices of 4 floats per token) for tokens below rope_count; V gets the
 * bias.  The fp16 results go to the packed Q / K / V images (n_heads regions
 * of token_tiles * head_dim * 32 halfwords) at token tiles out_offset/32 ..;
 * rows past `tokens` in the last tile are zeros.  d_bias may be NULL (zero).
 * head_dim 64 or 128; outputs 16-byte aligned.
 */
int hb_qkv_post(uint16_t *d_q, uint16_t *d_k, uint16_t *d_v, const float *d_raw, const float *d_bias,
                const float *d_q_norm, const float *d_k_norm, const float *d_pe, int rope_offset, int rope_count,
                int tokens, int n_heads, int head_dim, int token_tiles, int out_offset, hb_stream s);

/*
 * The same opcodes in one GEMM (reference src/dsp/ops/mat_mul.c:1373-1502,
 * the chunked HMX product with the post-processing of each output chunk):
 * d_x (tokens x input_dim f32) times the hb_f16_prepack image of the
 * input_dim x 3*n_heads*head_dim weight, with the post-processing of
 * hb_qkv_post applied to each 128 x 128 output tile in LDS, so the f32
 * product never reaches HBM.  Results are identical to hb_f16_gemm_ws (mode
 * 0, no bias) followed by hb_qkv_post.  n_heads * head_dim must be a
 * multiple of 128; d_workspace (256-byte aligned) holds
 * hb_qkv_gemm_workspace_bytes(tokens, input_dim) bytes, no state.
 */
size_t hb_qkv_gemm_workspace_bytes(int tokens, int input_dim);
int hb_qkv_gemm(uint16_t *d_q, uint16_t *d_k, uint16_t *d_v, const float *d_x, const uint16_t *d_packed,
                const float *d_bias, const float *d_q_norm, const float *d_k_norm, const float *d_pe, int rope_offset,
                int rope_count, int tokens, int input_dim, int n_heads, int head_dim, int token_tiles, int out_offset,
                void *d_workspace, size_t workspace_bytes, hb_stream s);

#ifdef __cplusplus
}
#endif

#endif /* HTP_OPS_HB_H */
