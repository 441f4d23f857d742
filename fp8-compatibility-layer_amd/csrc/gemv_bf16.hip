// GEMV instantiations for bf16 activations (one translation unit per activation dtype).
#include "gemv_impl.h"

namespace tfp8 {

void run_gemv_bf16(const void* x, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind, int G, int fmt,
                  const float* bias, void* y, int y_dtype, int ng, int gshift, hipStream_t s) {
    TFP8_DISPATCH_FMT(fmt, F, {
        if (ng > 1) launch_gemv_m<TFP8_BF16, F, true>(x, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, s);
        else launch_gemv_m<TFP8_BF16, F, false>(x, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, s);
    });
}

}  // namespace tfp8
