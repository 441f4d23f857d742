// Row-pair GEMV (the kernel is in gemv_pair_impl.h): the 1, 2 and 4 KB-chunk instantiations
// (K = 2048, 4096, 8192: the C1 and C2 shapes), the waves-per-block choice and the routing.
#include "gemv_pair_impl.h"

namespace tfp8 {

// Waves (row pairs) per block: 8 when a grid of 8-wave blocks is one block per CU (7/8 of the CUs
// or more busy), else 4.  Measured on MI355X (256 CUs), us per launch: C1 (2048 pairs) 8 per block
// 4.36, 4 per block 4.63; C2 M=1 (7168 pairs) 4 per block 10.56, 8 per block 10.92; 7, 14 or 16 per
// block were slower for both (5.3-5.9 and 11.1-12.1).
int pair_waves_per_block(int pairs) {
    const int forced = tune(TUNE_GEMV_PAIR);
    if (forced == 4 || forced == 8) return forced;
    const long cus = dev_info().cus;
    const long nblk8 = (pairs + 7) / 8;
    return nblk8 <= cus && nblk8 * 8 >= cus * 7 ? 8 : 4;
}

// The other chunk counts (gemv_pair_k.hip); false where (cpr, M) has no instantiation.
bool pair_other_cpr(int cpr, int M);
void launch_pair_other(int cpr, int x_dtype, int fmt, int M, int L, bool ue8, const void* x, const uint8_t* w,
                       const void* ws, const float* bias, void* y, int ydt, int N, int K, hipStream_t s);

// Runs the pair GEMV if it takes the shape (1 <= M <= pair_max_m(), f16/bf16 x, K % 16 == 0 with
// K = 2048, 4096, 8192 or ceil(K / 1024) chunks of 3, 5, 6, 7 (or 11, 12 for M <= 2), one scale per row or
// K-groups of 64/128/256 that the
// chunks cover, weights below 2^31 bytes, y aligned for the pair store); returns NOT_TAKEN otherwise.
int run_gemv_pair(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                  int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    if (M < 1 || M > tune(TUNE_GEMV_PAIR_MAX_M) || M > 4 || x_dtype == TFP8_F32 || !tune(TUNE_GEMV_PAIR))
        return NOT_TAKEN;
    const int cpr = (K + GEMV_CHUNK - 1) / GEMV_CHUNK;
    const bool here = (cpr == 2 || cpr == 4 || cpr == 8) && K == cpr * GEMV_CHUNK;   // compile-time K
    if (K % 16 || (!here && !pair_other_cpr(cpr, M)) || (long)N * K >= (1L << 31)) return NOT_TAKEN;
    int L = 0;
    if (G != K) {
        L = G / 16;
        if ((L != 4 && L != 8 && L != 16) || L < cpr || K % G) return NOT_TAKEN;
    }
    if ((uintptr_t)y % (y_dtype == TFP8_F32 ? 8 : 4) || (M > 1 && N % 2)) return NOT_TAKEN;
    const bool ue8 = ws_kind == TFP8_SCALE_UE8M0;
    if (!here) {
        launch_pair_other(cpr, x_dtype, fmt, M, L, ue8, x, w, ws, bias, y, y_dtype, N, K, s);
        return check_launch("tfp8_gemv (pair)");
    }
// K known at compile time, except at two activation rows, where the run-time-K form measured faster
// (C2 M=2: 11.15-11.24 vs 11.41-11.48 us, same box; C1 and C2 M=1 the other way round, 4.44 vs 4.39).
#define TFP8_PAIR_CPR(XD, F, MT)                                                                          \
    {                                                                                                    \
        if (cpr == 2) launch_pair_l<XD, F, 2, MT, MT != 2>(L, ue8, x, w, ws, bias, y, y_dtype, M, N, K, s);       \
        else if (cpr == 4) launch_pair_l<XD, F, 4, MT, MT != 2>(L, ue8, x, w, ws, bias, y, y_dtype, M, N, K, s);  \
        else launch_pair_l<XD, F, 8, MT, MT != 2>(L, ue8, x, w, ws, bias, y, y_dtype, M, N, K, s);               \
    }
#define TFP8_PAIR_M(XD, F)                                  \
    {                                                      \
        if (M == 1) TFP8_PAIR_CPR(XD, F, 1)                \
        else if (M == 2) TFP8_PAIR_CPR(XD, F, 2)           \
        else TFP8_PAIR_CPR(XD, F, 4)                       \
    }
    if (x_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_PAIR_M(TFP8_BF16, F));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_PAIR_M(TFP8_F16, F));
    }
#undef TFP8_PAIR_M
#undef TFP8_PAIR_CPR
    return check_launch("tfp8_gemv (pair)");
}

}  // namespace tfp8
