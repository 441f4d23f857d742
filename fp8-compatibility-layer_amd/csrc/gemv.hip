// Streaming FP8-weight GEMV for M <= 8 rows (the decode step).
//
// y[m,n] = sum_c s(n, c) * sum_{t<16} x[m, c+t] * decode(w[n, c+t]) + bias[n]   (c = 16-chunks)
// which is the formula of the reference GEMV (tfp8/csrc/tfp8_kernels.cu:171-269), laid out for
// CDNA4 instead of 32-lane warps:
//   * a 16-lane DPP row owns R weight rows; lane j streams the 16-byte chunks k = 16j + 256i of
//     each row with one global_load_dwordx4, so a row is read as 256 contiguous bytes per step
//     and a wave (4 DPP rows) touches 4R rows at once;
//   * U steps are issued before any of them is consumed, so R*U dwordx4 loads are in flight per
//     lane (all of the weight stream for a 4096-wide layer at the default shapes);
//   * codes are decoded in registers with v_cvt_pk_f32_fp8/bf8 (2 codes per instruction), no
//     LDS table; activations are read in their own dtype straight from global memory (every
//     DPP row of a wave reads the same addresses, so they coalesce) and converted to fp32;
//   * fp32 FMA accumulation; a K-group scale multiplies each 16-chunk partial, a per-channel
//     scale multiplies the final sum; the 16 lanes of a row are reduced with 4 DPP adds
//     (quad_perm x2, row_half_mirror, row_mirror) and lane m writes output row m.
#include "tfp8_common.h"

namespace tfp8 {

constexpr int GEMV_THREADS = 256;            // 4 waves = 16 DPP rows per block
constexpr int GEMV_ROWS_PER_BLOCK_GROUPS = GEMV_THREADS / 16;

template <int XDT>
__device__ __forceinline__ void load_x16(const void* __restrict__ x, size_t off, float* o) {
    if constexpr (XDT == TFP8_F32) {
        const float4* p = (const float4*)((const float*)x + off);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4 v = p[t];
            o[4 * t] = v.x; o[4 * t + 1] = v.y; o[4 * t + 2] = v.z; o[4 * t + 3] = v.w;
        }
    } else {
        const uint4* p = (const uint4*)((const uint16_t*)x + off);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 v = p[h];
            const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if constexpr (XDT == TFP8_BF16) {
                    o[8 * h + 2 * t] = __uint_as_float(d[t] << 16);
                    o[8 * h + 2 * t + 1] = __uint_as_float(d[t] & 0xFFFF0000u);
                } else {
                    o[8 * h + 2 * t] = f16_bits_to_f32(d[t] & 0xFFFFu);
                    o[8 * h + 2 * t + 1] = f16_bits_to_f32(d[t] >> 16);
                }
            }
        }
    }
}

template <int MT, int XDT, int FMT, bool GROUPED, int R, int U>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(
    const void* __restrict__ x, const uint8_t* __restrict__ w, const void* __restrict__ ws, int sk,
    const float* __restrict__ bias, void* __restrict__ y, int ydt, int M, int N, int K, int G, int ng,
    int gshift) {
    const int j = threadIdx.x & 15;
    const int grp = blockIdx.x * GEMV_ROWS_PER_BLOCK_GROUPS + (threadIdx.x >> 4);
    const int n0 = grp * R;
    if (n0 >= N) return;   // uniform over the 16-lane row

    const uint8_t* wp[R];
    size_t srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(n0 + r, N - 1);   // rows past N re-read the last row; never stored
        wp[r] = w + (size_t)n * K;
        srow[r] = (size_t)n * ng;
    }

    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

    for (int kb = 16 * j; kb < K; kb += 256 * U) {
        uint4 wv[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = kb + 256 * u;
#pragma unroll
            for (int r = 0; r < R; ++r)
                wv[u][r] = k < K ? *(const uint4*)(wp[r] + k) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = kb + 256 * u;
            if (k < K) {
                float xf[MT][16];
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    if (m < M) load_x16<XDT>(x, (size_t)m * K + k, xf[m]);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float wf[16];
                    dec4_f32<FMT>(wv[u][r].x, wf);
                    dec4_f32<FMT>(wv[u][r].y, wf + 4);
                    dec4_f32<FMT>(wv[u][r].z, wf + 8);
                    dec4_f32<FMT>(wv[u][r].w, wf + 12);
                    float s = 1.f;
                    if constexpr (GROUPED) {
                        const int g = gshift >= 0 ? (k >> gshift) : (k / G);
                        s = sk == TFP8_SCALE_UE8M0 ? ue8m0_to_f32(((const uint8_t*)ws)[srow[r] + g])
                                                   : ((const float*)ws)[srow[r] + g];
                    }
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m < M) {
                            if constexpr (GROUPED) {
                                float p = 0.f;
#pragma unroll
                                for (int t = 0; t < 16; ++t) p = fmaf(xf[m][t], wf[t], p);
                                acc[r][m] = fmaf(p, s, acc[r][m]);
                            } else {
                                float a = acc[r][m];
#pragma unroll
                                for (int t = 0; t < 16; ++t) a = fmaf(xf[m][t], wf[t], a);
                                acc[r][m] = a;
                            }
                        }
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        float s = 1.f;
        if constexpr (!GROUPED)
            s = sk == TFP8_SCALE_UE8M0 ? ue8m0_to_f32(((const uint8_t*)ws)[srow[r]]) : ((const float*)ws)[srow[r]];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = row16_sum(acc[r][m]) * s;
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = n0 + r;
        float v = acc[r][0];
#pragma unroll
        for (int m = 1; m < MT; ++m) v = (j == m) ? acc[r][m] : v;
        if (n < N && j < M) {
            const float b = bias ? bias[n] : 0.f;
            store_elem(y, (size_t)j * N + n, ydt, v + b);
        }
    }
}

struct GemvCfg { int R, U; };

// Rows per DPP row (R) and steps in flight (U) by row-tile height.  Chosen by a sweep on
// MI355X; every shape is correct with any of them.
static GemvCfg gemv_cfg(int MT) {
    if (MT <= 2) return {2, 4};
    return {4, 2};
}

template <int MT, int XDT, int FMT, bool GROUPED>
static void launch_gemv_t(const void* x, const uint8_t* w, const void* ws, int sk, const float* bias, void* y,
                          int ydt, int M, int N, int K, int G, int ng, int gshift, hipStream_t s) {
    const GemvCfg c = gemv_cfg(MT);
    if (c.R == 2) {
        constexpr int R = 2, U = 4;
        const unsigned grid = (unsigned)((N + GEMV_ROWS_PER_BLOCK_GROUPS * R - 1) / (GEMV_ROWS_PER_BLOCK_GROUPS * R));
        gemv_kernel<MT, XDT, FMT, GROUPED, R, U><<<grid, GEMV_THREADS, 0, s>>>(x, w, ws, sk, bias, y, ydt, M, N, K,
                                                                              G, ng, gshift);
    } else {
        constexpr int R = 4, U = 2;
        const unsigned grid = (unsigned)((N + GEMV_ROWS_PER_BLOCK_GROUPS * R - 1) / (GEMV_ROWS_PER_BLOCK_GROUPS * R));
        gemv_kernel<MT, XDT, FMT, GROUPED, R, U><<<grid, GEMV_THREADS, 0, s>>>(x, w, ws, sk, bias, y, ydt, M, N, K,
                                                                              G, ng, gshift);
    }
}

template <int XDT, int FMT, bool GROUPED>
static void launch_gemv_m(const void* x, const uint8_t* w, const void* ws, int sk, const float* bias, void* y,
                          int ydt, int M, int N, int K, int G, int ng, int gshift, hipStream_t s) {
    if (M <= 1) launch_gemv_t<1, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
    else if (M <= 2) launch_gemv_t<2, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
    else if (M <= 4) launch_gemv_t<4, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
    else launch_gemv_t<8, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
}

// Validated by the caller (linear.hip).  1 <= M <= 8.
int run_gemv(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind, int G,
             int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    const int ng = K / G;
    const bool grouped = ng > 1;
    int gshift = -1;
    if ((G & (G - 1)) == 0) gshift = __builtin_ctz((unsigned)G);
    TFP8_DISPATCH_DT(x_dtype, D, TFP8_DISPATCH_FMT(fmt, F, {
        if (grouped) launch_gemv_m<D, F, true>(x, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, s);
        else launch_gemv_m<D, F, false>(x, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, s);
    }));
    return check_launch("tfp8_gemv");
}

}  // namespace tfp8
