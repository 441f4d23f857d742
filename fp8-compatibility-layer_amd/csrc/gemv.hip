// GEMV entry: validated by the caller (linear.hip), 1 <= M <= 8.  In order of preference: the
// 4x4x4-MFMA GEMV (gemv_quad.hip), the row-pair GEMV (gemv_pair.hip), the matrix-core decode kernel
// (gemv_mfma.hip, from TFP8_GEMV_MFMA_MIN rows), and the streaming GEMV (gemv_impl.h, dispatched
// by activation dtype), each taking the shapes it was measured best on and returning NOT_TAKEN
// otherwise.
#include "tfp8_common.h"

namespace tfp8 {

void run_gemv_f16(const void*, int, int, const uint8_t*, int, const void*, int, int, int, const float*, void*, int, int,
                  int, hipStream_t);
void run_gemv_bf16(const void*, int, int, const uint8_t*, int, const void*, int, int, int, const float*, void*, int,
                   int, int, hipStream_t);
void run_gemv_f32(const void*, int, int, const uint8_t*, int, const void*, int, int, int, const float*, void*, int, int,
                  int, hipStream_t);

int run_gemv_pair(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                  int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s);
int run_gemv_quad(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                  int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s);
int run_gemv_mfma(const void* x, int x_dtype, const float* xs, int M, int K, const uint8_t* w, int N, const void* ws,
                  int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s);

// Smallest M that goes to the matrix-core decode kernel (gemv_mfma.hip); below it the streaming
// GEMV's per-row dot products are cheaper (measured on MI355X: C2 M=2 12.5 vs 17.1 us, M=4
// 19.3 vs 17.9 us, M=8 35.2 vs 19.2 us).  Knob TFP8_GEMV_MFMA_MIN (default 4).
int gemv_mfma_min_m() { return tune(TUNE_GEMV_MFMA_MIN); }

int run_gemv(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind, int G,
             int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    {
        const int rc = run_gemv_quad(x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, s);
        if (rc != NOT_TAKEN) return rc;
    }
    {
        const int rc = run_gemv_pair(x, x_dtype, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, s);
        if (rc != NOT_TAKEN) return rc;
    }
    if (M >= gemv_mfma_min_m()) {
        const int rc = run_gemv_mfma(x, x_dtype, nullptr, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, s);
        if (rc != NOT_TAKEN) return rc;
    }
    const int ng = K / G;
    int gshift = -1;
    if ((G & (G - 1)) == 0) gshift = __builtin_ctz((unsigned)G);
    if (x_dtype == TFP8_F16) run_gemv_f16(x, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, ng, gshift, s);
    else if (x_dtype == TFP8_BF16) run_gemv_bf16(x, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, ng, gshift, s);
    else run_gemv_f32(x, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, ng, gshift, s);
    return check_launch("tfp8_gemv");
}

}  // namespace tfp8
