/*
 * tfp8_hip.h -- C ABI of libtfp8_hip.so, the MI355X (gfx950) kernels behind the tfp8
 * FP8Linear fused-dequant path.
 *
 * Every entry point is a plain host function: device pointers, sizes, enum codes and a
 * hipStream_t passed as void*.  Nothing here allocates or frees device memory, nothing
 * synchronises the host, and every launch is ordered on the given stream.  A return value of 0
 * means the work was enqueued; a negative value is an argument error detected on the host
 * before anything was launched; a positive value is a hipError_t from the launch.  The message
 * for the last failure on the calling thread is returned by tfp8_last_error().
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   tfp8/_ext.py:45-76      available()/_get(): NVRTC compile + module load per device
 *   tfp8/_ext.py:132-157    _launch(): ctypes cuLaunchKernel with cached argument slots
 *   tfp8/_ext.py:230-253    w8a16(): M<=8 GEMV / M>8 GEMM dispatch          -> tfp8_linear
 *   tfp8/_ext.py:163-217    GemvLaunch (kernels tfp8_gemv_in_*_m*_*)         -> tfp8_gemv
 *   tfp8/_ext.py:259-275    _gemm_launch()/gemm_prepared() (tfp8_gemm_*)     -> tfp8_gemm_prepared
 *   tfp8/_ext.py:220-227    prepare_activations() (tfp8_prep_*)              -> tfp8_prepare_activations
 *   tfp8/_ext.py:305-315    dequant_into() (tfp8_dequant_f16)                -> tfp8_dequant
 *   tfp8/formats.py:43-69   decode()/lut() (torch, CPU/CUDA)                 -> tfp8_decode
 *   tfp8/formats.py:77-96   encode() (torch, CPU/CUDA)                       -> tfp8_encode
 *   tfp8/quantize.py:15-36  quantize_weight() (torch)                        -> tfp8_quantize_weight
 *   fp8_cuda.py:85-88 + fp8_gemm_kernel.cu:22-30  UE8M0 scale encode/decode rule (scale_kind 1)
 */
#ifndef TFP8_HIP_H
#define TFP8_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TFP8_ABI_VERSION 1

/* Element types of activations, outputs and decoded values. */
enum tfp8_dtype { TFP8_F16 = 0, TFP8_BF16 = 1, TFP8_F32 = 2 };
/* FP8 code formats (tfp8/formats.py:30-31; FMT_ID in tfp8/_ext.py:41). */
enum tfp8_fmt { TFP8_E4M3FN = 0, TFP8_E5M2 = 1 };
/* Weight-scale storage: fp32 values, or UE8M0 bytes meaning 2^(b-127), 255 = NaN. */
enum tfp8_scale_kind { TFP8_SCALE_F32 = 0, TFP8_SCALE_UE8M0 = 1 };

/* Error codes returned before any launch. */
#define TFP8_ERR_ARG (-1)      /* bad size, enum or null pointer */
#define TFP8_ERR_ALIGN (-2)    /* pointer or stride not aligned as required */
#define TFP8_ERR_SHAPE (-3)    /* K/G divisibility the kernels require */
#define TFP8_ERR_WORKSPACE (-4) /* workspace missing or too small */

/* Version of this ABI (TFP8_ABI_VERSION). */
int tfp8_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char* tfp8_last_error(void);

/*
 * out[i] = decode(q[i]) for i < n, written as f16/bf16/f32.  Exact for every code; NaN codes
 * give a NaN, E5M2 0x7C/0xFC give +-inf.  Replaces formats.decode / formats.lut
 * (tfp8/formats.py:43-69).  No alignment requirement.
 */
int tfp8_decode(const uint8_t* q, int64_t n, int fmt, void* out, int out_dtype, void* stream);

/*
 * q[i] = encode(x[i]): round-to-nearest-even, saturating to +-max_finite (never inf), NaN ->
 * 0x7F (E4M3FN) / 0x7E (E5M2).  Same rule as formats.encode (tfp8/formats.py:77-96) and
 * fp8.h:55-76 apart from the NaN code, which follows formats.py:94-95.
 */
int tfp8_encode(const void* x, int x_dtype, int64_t n, int fmt, uint8_t* q, void* stream);

/*
 * Symmetric weight quantisation, tfp8/quantize.py:15-36: for each row n and K-group g of w
 * [N,K] (row-major, x_dtype elements), amax = max|w|, s = max(amax/max_finite, FLT_MIN),
 * s = 2^ceil(log2 s) when pow2 (always for UE8M0), s = 1 when amax == 0, then
 * q = encode(clamp(w/s, +-max_finite)).  scale is f32 [N, K/G] or, for TFP8_SCALE_UE8M0,
 * uint8 [N, K/G] holding ceil(log2 s)+127 clamped to [0,254] (fp8_cuda.py:85-88).
 * K % G == 0 required.
 */
int tfp8_quantize_weight(const void* w, int w_dtype, int N, int K, int G, int fmt, int pow2,
                         int scale_kind, uint8_t* q, void* scale, void* stream);

/*
 * Activation row preparation for fp16 MFMA, tfp8/quantize.py:47-62 and _ext.py:220-227:
 * per row, e = ceil(log2 amax) - 8 (0 if amax == 0, exact from the exponent bits),
 * x16 = fp16(x / 2^e), xs = 2^e.  x is [M,K] f16/bf16/f32, x16 is [M,K] fp16, xs is [M] f32.
 */
int tfp8_prepare_activations(const void* x, int x_dtype, int M, int K, void* x16, float* xs,
                             void* stream);

/*
 * Weight dequantisation into a caller buffer, out[n,k] = decode(w[n,k]) * scale(n, k/G), in
 * f16/bf16/f32 (f32 is exact).  Replaces _ext.dequant_into / tfp8_dequant_f16
 * (tfp8/_ext.py:305-315); used by tests and the module's numeric fallback, never by the
 * forward hot path.
 */
int tfp8_dequant(const uint8_t* w, int N, int K, const void* ws, int ws_kind, int G, int fmt,
                 void* out, int out_dtype, void* stream);

/*
 * y[m,n] = sum_k x[m,k] * decode(w[n,k]) * scale(n, k/G) + bias[n]  (fp32 accumulation),
 * the FP8Linear forward (tfp8/linear.py:150-208 through _ext.w8a16, tfp8/_ext.py:230-253).
 *
 *   x     [M,K] row-major, x_dtype; 16-byte aligned
 *   w     [N,K] uint8 FP8 codes row-major; 16-byte aligned, K % 16 == 0
 *   ws    [N,K/G] f32 or UE8M0 bytes (ws_kind); G % 16 == 0, K % G == 0
 *   bias  [N] f32 or NULL
 *   y     [M,N] row-major, y_dtype
 *
 * M <= 8 runs the GEMV path: the 4x4x4-MFMA GEMV for 3-8 f16/bf16 rows with one scale per row
 * (3-4 rows with K groups of 64, 128 or 256) and K = 2048 or 4096; the row-pair GEMV for 1-4
 * f16/bf16 rows when K is 2048, 4096 or 8192, or K / 1024 rounded up is 3, 5, 6 or 7 (11 or 12 for
 * 1-2 rows), G == K or G is 64,
 * 128 or 256 (G >= 16 * that chunk count), and N is even for M > 1; otherwise the
 * streaming GEMV up to 3 rows and the matrix-core decode kernel from 4.  M > 8 runs the MFMA
 * GEMM path (the decode kernel up to 16 rows, then the weight-streaming, direct-to-LDS or
 * LDS-tiled GEMM by M and scale layout), which additionally needs G == K or G % 32 == 0.  fp32 activations on the GEMM path are first converted to
 * fp16 with a power-of-two row scale (tfp8_prepare_activations) in the workspace; the GEMM
 * may also split K across blocks and keep fp32 partial sums there.  The needed size is
 * tfp8_linear_workspace_size(); pass NULL/0 when it returns 0.  M == 0 is a no-op.
 */
size_t tfp8_linear_workspace_size(int x_dtype, int M, int N, int K);
int tfp8_linear(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N,
                const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y,
                int y_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * tfp8_linear without a caller workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  Same arguments, routing, kernels and results as tfp8_linear; its split-K
 * partial sums and fp32-activation staging go to a library-owned scratch array of
 * TFP8_NOALLOC_SCRATCH_BYTES per GPU (held from library load until the process ends), so it calls
 * no hipMalloc/hipFree.  A shape whose tfp8_linear_workspace_size() exceeds that returns
 * TFP8_ERR_WORKSPACE without launching.  All calls on one GPU share its scratch: calls that
 * overlap on one GPU (several streams or host threads at once) race and must be serialised by the
 * caller; calls in order on one stream are safe.  The first call with a device current resolves
 * that device's scratch address (hipGetSymbolAddress) -- make that call outside graph capture.
 */
#define TFP8_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int tfp8_linear_noalloc(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N,
                        const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y,
                        int y_dtype, void* stream);

/* The GEMV alone (1 <= M <= 8), any x_dtype; GEMV kernels of tfp8/csrc/tfp8_kernels.cu:171-269. */
int tfp8_gemv(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N,
              const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y,
              int y_dtype, void* stream);

/*
 * The MFMA GEMM alone on f16 or bf16 activations, with an optional per-row f32 scale xs [M]
 * (NULL = 1), i.e. _ext.gemm_prepared (tfp8/_ext.py:267-275) / gemm_w8a16
 * (tfp8/csrc/tfp8_kernels.cu:296-411).  Any M >= 1 (M <= 8 runs the GEMM kernels too, not the
 * GEMV).  The workspace (split-K partial sums) must hold tfp8_gemm_prepared_workspace_size(M, N, K)
 * bytes, 256-byte aligned; that size can be non-zero for every M, including M <= 8.
 */
size_t tfp8_gemm_prepared_workspace_size(int x16_dtype, int M, int N, int K);
int tfp8_gemm_prepared(const void* x16, int x16_dtype, const float* xs, int M, int K,
                       const uint8_t* w, int N, const void* ws, int ws_kind, int G, int fmt,
                       const float* bias, void* y, int y_dtype, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- tuning knobs
 * No counterpart in the reference (its kernels are resolved once per device, tfp8/_ext.py:67-76).
 * Kernel-selection overrides for sweeps and for tests that force every compiled configuration:
 * TFP8_GEMV_CFG, TFP8_GEMV_WPC, TFP8_GEMV_MFMA_MIN, TFP8_GEMV_MFMA_MAX_M, TFP8_GM_NT, TFP8_GM_W,
 * TFP8_GM_D, TFP8_GM_TL, TFP8_GEMM_TILE, TFP8_GEMM_SPLITK, TFP8_GEMM_DIRECT, TFP8_GEMM_DIRECT_MIN_M,
 * TFP8_GEMM_DCFG, TFP8_GS_NW, TFP8_GS_KCS, TFP8_GS_SPLITK, TFP8_GS_TL, TFP8_GEMM_V1, TFP8_GEMV_PAIR,
 * TFP8_GEMV_PAIR_MAX_M, TFP8_GEMV_QUAD, TFP8_GEMV_QUAD_MIN_M.  Each starts at the value of the
 * environment variable of that name when the library is loaded (or its default), and changes only
 * through tfp8_tuning_set; the launch path never reads the environment.  A knob
 * changes routing and workspace sizes for every later call in the process: size workspaces after
 * setting knobs.  tfp8_tuning_reset restores the values read at load.  Unknown names give
 * TFP8_ERR_ARG.
 */
int tfp8_tuning_set(const char* name, int value);
int tfp8_tuning_get(const char* name, int* value);
void tfp8_tuning_reset(void);

/* ---------------------------------------------------------------- W8A8, 32-wide K-block scales
 * FP8 activations x FP8 weights (reference fp8_cuda.py / fp8_gemm_kernel.cu).
 *
 * tfp8_w8a8_quantize replaces fp8_cuda.quantize_k (fp8_cuda.py:74-92): x [R, K] (f16/bf16/f32,
 * K % 32 == 0) -> q [R, K] FP8 codes (16-byte aligned) and per (row, 32-block) scales [R, K/32]:
 * s = max(amax / max_finite, 1e-12), f32; or with ue8m0, e = clamp(ceil(log2 s), -127, 127), the
 * byte e + 127 and s = 2^e.  q = encode(clamp(x / s, +-max_finite)) (round to nearest even).
 */
int tfp8_w8a8_quantize(const void* x, int x_dtype, int R, int K, int fmt, int ue8m0, uint8_t* q, void* scale,
                       void* stream);

/* tfp8_w8a8_gemm replaces the gemm_block_* / gemm_rowcol_* kernels (fp8_gemm_kernel.cu:41-118,
 * launched by fp8_cuda.fp8_linear, fp8_cuda.py:109-138):
 *   mode 0 (block):   C[m,n] = sum_kb sa[m,kb] * sb[n,kb] * sum_{k in kb} A[m,k] Bt[n,k] + bias[n]
 *                     sa [M, K/32], sb [N, K/32]
 *   mode 1 (row/col): C[m,n] = (sum_k A[m,k] Bt[n,k]) * sa[m] * sb[n] + bias[n];  sa [M], sb [N]
 * A [M, K] codes in fmt_a, Bt [N, K] codes in fmt_b (the weight transposed: k contiguous); scales
 * f32, or UE8M0 bytes (255 = NaN) with ue8m0; bias f32 [N] or NULL; C f32 [M, N].  K % 32 == 0;
 * A and Bt 16-byte aligned.  (The reference requires M, N, K % 32 == 0; any M, N work here.)
 * native_fp8 = 0: codes decoded to f16 and multiplied on f16 matrix cores, products exact in the
 *   fp32 sums (the reference's fp16 WMMA numerics; max|C - C64| / max|C64| ~ 1e-7).
 * native_fp8 = 1: FP8 matrix cores (UE8M0 block scales applied by the MX-scaled instruction);
 *   those align each dot product's terms to the largest, so ~1e-5 .. 1e-4 of max|C|.
 */
int tfp8_w8a8_gemm(const uint8_t* a, int fmt_a, const void* sa, const uint8_t* bt, int fmt_b, const void* sb,
                   int ue8m0, int mode, int native_fp8, const float* bias, float* c, int M, int N, int K,
                   void* stream);

/* ---------------------------------------------------------------- measurement
 * No counterpart in the reference: a plain read-only streaming kernel for the measurement harness
 * (a reference rate beside the GEMV's).  Reads `bytes` (a multiple of 16, 16-byte aligned)
 * of p with `blocks` blocks of 512 threads and stores each block's XOR of the 32-bit words it read
 * in out[block] (blocks <= 65536); the XOR over out[] is the XOR of every word of the buffer.
 */
int tfp8_read_probe(const void* p, size_t bytes, uint32_t* out, int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TFP8_HIP_H */
