// Row-pair GEMV (the kernel is in gemv_pair_impl.h) for K that is not 2048, 4096 or 8192: 3, 5, 6, 7,
// 11 and 12 chunks of 1 KB per row (the last one partial when K % 1024 != 0; above 8 chunks up to two
// activation rows, whose x fits the block's LDS), which covers LLM down projections at decode such as
// K = 5632 and 11008, and K = 3072, 6144, 12288.  Same box, us, this kernel vs the streaming GEMV /
// matrix-core decode kernel it replaces: M=1 2048x5632 3.88 vs 5.35, 4096x11008 10.49 vs 12.18, M=2
// 4096x11008 10.32 vs 13.31, M=4 2048x5632 5.26 vs 8.17, M=1 4096x5632 G=128 5.90 vs 7.33.  14 chunks
// (K = 13824, 14336: 175 VGPRs) only tied the streaming GEMV (12.53 vs 12.36) and is not built.
// Compiled apart from gemv_pair.hip so that the two build in parallel.
#include "gemv_pair_impl.h"

namespace tfp8 {

bool pair_other_cpr(int cpr, int M) {
    return cpr == 3 || cpr == 5 || cpr == 6 || cpr == 7 || ((cpr == 11 || cpr == 12) && M <= 2);
}

void launch_pair_other(int cpr, int x_dtype, int fmt, int M, int L, bool ue8, const void* x, const uint8_t* w,
                       const void* ws, const float* bias, void* y, int ydt, int N, int K, hipStream_t s) {
#define TFP8_PAIRK_CPR(XD, F, MT)                                                                          \
    {                                                                                                     \
        switch (cpr) {                                                                                    \
            case 3: launch_pair_l<XD, F, 3, MT, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;       \
            case 5: launch_pair_l<XD, F, 5, MT, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;       \
            case 6: launch_pair_l<XD, F, 6, MT, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;       \
            case 7: launch_pair_l<XD, F, 7, MT, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;       \
            case 11: launch_pair_l<XD, F, 11, MT, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;     \
            default: launch_pair_l<XD, F, 12, MT, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;     \
        }                                                                                                 \
    }
// Four activation rows only up to 8 chunks (x of the block within 64 KB of LDS).
#define TFP8_PAIRK_CPR4(XD, F)                                                                            \
    {                                                                                                     \
        switch (cpr) {                                                                                    \
            case 3: launch_pair_l<XD, F, 3, 4, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;        \
            case 5: launch_pair_l<XD, F, 5, 4, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;        \
            case 6: launch_pair_l<XD, F, 6, 4, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;        \
            default: launch_pair_l<XD, F, 7, 4, false>(L, ue8, x, w, ws, bias, y, ydt, M, N, K, s); break;       \
        }                                                                                                 \
    }
#define TFP8_PAIRK_M(XD, F)                                 \
    {                                                      \
        if (M == 1) TFP8_PAIRK_CPR(XD, F, 1)               \
        else if (M == 2) TFP8_PAIRK_CPR(XD, F, 2)          \
        else TFP8_PAIRK_CPR4(XD, F)                        \
    }
    if (x_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_PAIRK_M(TFP8_BF16, F));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_PAIRK_M(TFP8_F16, F));
    }
#undef TFP8_PAIRK_M
#undef TFP8_PAIRK_CPR4
#undef TFP8_PAIRK_CPR
}

}  // namespace tfp8
