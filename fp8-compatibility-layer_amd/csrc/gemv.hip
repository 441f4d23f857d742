// GEMV entry: validated by the caller (linear.hip), 1 <= M <= 8; dispatch by activation dtype.
// The kernel and its launch configurations are in gemv_impl.h.
#include "tfp8_common.h"

namespace tfp8 {

void run_gemv_f16(const void*, int, int, const uint8_t*, int, const void*, int, int, int, const float*, void*, int, int,
                  int, hipStream_t);
void run_gemv_bf16(const void*, int, int, const uint8_t*, int, const void*, int, int, int, const float*, void*, int,
                   int, int, hipStream_t);
void run_gemv_f32(const void*, int, int, const uint8_t*, int, const void*, int, int, int, const float*, void*, int, int,
                  int, hipStream_t);

int run_gemv(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind, int G,
             int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    const int ng = K / G;
    int gshift = -1;
    if ((G & (G - 1)) == 0) gshift = __builtin_ctz((unsigned)G);
    if (x_dtype == TFP8_F16) run_gemv_f16(x, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, ng, gshift, s);
    else if (x_dtype == TFP8_BF16) run_gemv_bf16(x, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, ng, gshift, s);
    else run_gemv_f32(x, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, ng, gshift, s);
    return check_launch("tfp8_gemv");
}

}  // namespace tfp8
