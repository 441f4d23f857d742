// FP8Linear entry points: argument validation, path selection by M (GEMV for M <= 8, MFMA GEMM
// above, as tfp8/_ext.py:230-253 routes), workspace layout.
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "tfp8_common.h"

namespace tfp8 {

int run_gemv(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind, int G,
             int fmt, const float* bias, void* y, int y_dtype, hipStream_t s);
int run_gemm(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
             const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, float* partial,
             hipStream_t s);
size_t gemm_partial_bytes(int M, int N, int K);

constexpr int GEMV_MAXM = 8;   // tfp8/_ext.py:37

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Shared validation of the linear arguments; `what` names the entry point in messages.
static int check_linear(const char* what, const void* x, int x_dtype, int M, int K, const uint8_t* w, int N,
                        const void* ws, int ws_kind, int G, int fmt, const void* y, int y_dtype, bool gemm) {
    if (M < 0 || N < 0 || K <= 0 || G <= 0)
        return fail(TFP8_ERR_ARG, "%s: bad sizes M=%d N=%d K=%d G=%d", what, M, N, K, G);
    if (!valid_dtype(x_dtype) || !valid_dtype(y_dtype) || !valid_fmt(fmt) || !valid_sk(ws_kind))
        return fail(TFP8_ERR_ARG, "%s: bad enum (x_dtype=%d y_dtype=%d fmt=%d ws_kind=%d)", what, x_dtype, y_dtype,
                    fmt, ws_kind);
    if (K % 16 || G % 16 || K % G)
        return fail(TFP8_ERR_SHAPE, "%s: need K %% 16 == 0, G %% 16 == 0, K %% G == 0 (K=%d G=%d)", what, K, G);
    if (gemm && G != K && G % 32)
        return fail(TFP8_ERR_SHAPE, "%s: the GEMM needs G == K or G %% 32 == 0 (G=%d)", what, G);
    if (M == 0 || N == 0) return 0;
    if (!x || !w || !ws || !y) return fail(TFP8_ERR_ARG, "%s: null pointer", what);
    if (!aligned(x, 16) || !aligned(w, 16))
        return fail(TFP8_ERR_ALIGN, "%s: x and w must be 16-byte aligned", what);
    if (ws_kind == TFP8_SCALE_F32 && !aligned(ws, 4)) return fail(TFP8_ERR_ALIGN, "%s: f32 scales misaligned", what);
    if (!aligned(y, y_dtype == TFP8_F32 ? 4 : 2)) return fail(TFP8_ERR_ALIGN, "%s: y misaligned", what);
    return 0;
}

}  // namespace tfp8

using namespace tfp8;

extern "C" size_t tfp8_linear_workspace_size(int x_dtype, int M, int N, int K) {
    if (M <= GEMV_MAXM || N <= 0 || K <= 0) return 0;
    size_t b = 0;
    if (x_dtype == TFP8_F32) b += align256((size_t)M * K * 2) + align256((size_t)M * 4);
    b += gemm_partial_bytes(M, N, K);
    return b;
}

extern "C" size_t tfp8_gemm_prepared_workspace_size(int x16_dtype, int M, int N, int K) {
    (void)x16_dtype;
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return gemm_partial_bytes(M, N, K);
}

extern "C" int tfp8_gemv(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws,
                         int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, void* stream) {
    clear_error();
    if (int rc = check_linear("tfp8_gemv", x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, y, y_dtype, false)) return rc;
    if (M > GEMV_MAXM) return fail(TFP8_ERR_ARG, "tfp8_gemv: M=%d exceeds %d", M, GEMV_MAXM);
    if (M == 0 || N == 0) return 0;
    return run_gemv(x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, (hipStream_t)stream);
}

extern "C" int tfp8_gemm_prepared(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w,
                                  int N, const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y,
                                  int y_dtype, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (x16_dtype != TFP8_F16 && x16_dtype != TFP8_BF16)
        return fail(TFP8_ERR_ARG, "tfp8_gemm_prepared: activations must be f16 or bf16");
    if (int rc = check_linear("tfp8_gemm_prepared", x16, x16_dtype, M, K, w, N, ws, ws_kind, G, fmt, y, y_dtype,
                              true))
        return rc;
    if (M == 0 || N == 0) return 0;
    const size_t need = gemm_partial_bytes(M, N, K);
    if (need && (!workspace || workspace_bytes < need || !aligned(workspace, 256)))
        return fail(TFP8_ERR_WORKSPACE, "tfp8_gemm_prepared: need %zu bytes of 256-aligned workspace, got %zu",
                    need, workspace ? workspace_bytes : (size_t)0);
    return run_gemm(x16, x16_dtype, xs, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, (float*)workspace,
                    (hipStream_t)stream);
}

// The body of tfp8_linear after validation, on a workspace already checked to be large enough.
static int linear_run(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                      int G, int fmt, const float* bias, void* y, int y_dtype, void* workspace, void* stream);

extern "C" int tfp8_linear(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws,
                           int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
    clear_error();
    const bool gemm = M > GEMV_MAXM;
    if (int rc = check_linear("tfp8_linear", x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, y, y_dtype, gemm))
        return rc;
    if (M == 0 || N == 0) return 0;
    const size_t need = gemm ? tfp8_linear_workspace_size(x_dtype, M, N, K) : 0;
    if (need && (!workspace || workspace_bytes < need || !aligned(workspace, 256)))
        return fail(TFP8_ERR_WORKSPACE, "tfp8_linear: need %zu bytes of 256-aligned workspace, got %zu", need,
                    workspace ? workspace_bytes : (size_t)0);
    return linear_run(x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, workspace, stream);
}

static int linear_run(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                      int G, int fmt, const float* bias, void* y, int y_dtype, void* workspace, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    if (M <= GEMV_MAXM) return run_gemv(x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, s);
    uint8_t* wsp = (uint8_t*)workspace;
    if (x_dtype == TFP8_F32) {
        // fp32 activations: fp16 with an exact power-of-two row scale (tfp8/quantize.py:47-62).
        void* x16 = wsp;
        float* xs = (float*)(wsp + align256((size_t)M * K * 2));
        float* part = (float*)(wsp + align256((size_t)M * K * 2) + align256((size_t)M * 4));
        if (int rc = tfp8_prepare_activations(x, x_dtype, M, K, x16, xs, stream)) return rc;
        return run_gemm(x16, TFP8_F16, xs, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, part, s);
    }
    return run_gemm(x, x_dtype, nullptr, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, (float*)wsp, s);
}

// ------------------------------------------------------------------ no-allocation entry point
// tfp8_linear for callers that cannot allocate (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc): the workspace is this file-scope device array instead of a
// caller buffer.  Each GPU holds its own copy, at its own address, from module load until the
// process ends.  Host code never passes `scratch` itself (in host code the name is a stand-in,
// not a device address): its address on each device comes from hipGetSymbolAddress, once per
// device, with that device current, and only that pointer is used.
namespace tfp8 {

constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;   // TFP8_NOALLOC_SCRATCH_BYTES in the header
static_assert(NOALLOC_SCRATCH_BYTES == TFP8_NOALLOC_SCRATCH_BYTES, "header and library agree on the limit");

__device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int SCRATCH_MAX_DEVICES = 64;
static std::atomic<void*> g_scratch[SCRATCH_MAX_DEVICES];
static std::mutex g_scratch_mu;

// The current device's copy of `scratch`, resolved on the first call made with that device current.
static int scratch_for_current_device(void** out) {
    int dev = -1;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) return fail((int)ge, "tfp8_linear_noalloc: hipGetDevice failed: %s", hipGetErrorString(ge));
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
        return fail(TFP8_ERR_ARG, "tfp8_linear_noalloc: device %d out of range", dev);
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return fail(e != hipSuccess ? (int)e : TFP8_ERR_ARG,
                            "tfp8_linear_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                            hipGetErrorString(e));
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return 0;
}

}  // namespace tfp8

extern "C" int tfp8_linear_noalloc(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws,
                                   int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype,
                                   void* stream) {
    clear_error();
    const bool gemm = M > GEMV_MAXM;
    if (int rc = check_linear("tfp8_linear_noalloc", x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, y, y_dtype, gemm))
        return rc;
    if (M == 0 || N == 0) return 0;
    const size_t need = gemm ? tfp8_linear_workspace_size(x_dtype, M, N, K) : 0;
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(TFP8_ERR_WORKSPACE,
                    "tfp8_linear_noalloc: M=%d N=%d K=%d needs %zu bytes of workspace, more than the %zu-byte "
                    "scratch; use tfp8_linear with a caller workspace",
                    M, N, K, need, NOALLOC_SCRATCH_BYTES);
    void* sp = nullptr;
    if (need)
        if (int rc = scratch_for_current_device(&sp)) return rc;
    // Nothing in the scratch needs clearing: split-K slices overwrite every partial they own and
    // the fp32-activation prep writes every fp16 value and row scale before they are read.
    return linear_run(x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, sp, stream);
}
