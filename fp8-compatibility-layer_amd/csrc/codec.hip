// Elementwise FP8 codec kernels: decode, encode (RNE, saturating), weight quantisation,
// activation row preparation and weight dequantisation.  All are HBM-streaming byte/element
// kernels; none of them is on the FP8Linear forward hot path except tfp8_prepare_activations
// (fp32 activations into the MFMA GEMM).
#include <float.h>

#include "tfp8_common.h"

namespace tfp8 {

constexpr int EW_THREADS = 256;
constexpr int EW_PER_THREAD = 4;

// ------------------------------------------------------------------ decode
// out[i] = decode(q[i]); four codes per thread assembled into one dword for the packed cvt.
// Follows tfp8/formats.py:43-57 (bit fields: subnormal m*2^(1-bias-mbits), normal
// (m+2^mbits)*2^(e-bias-mbits), E5M2 inf, NaN) via the hardware conversion.
template <int FMT, int ODT>
__global__ __launch_bounds__(EW_THREADS) void decode_kernel(const uint8_t* __restrict__ q, int64_t n,
                                                            void* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * EW_THREADS * EW_PER_THREAD;
    for (int64_t i = ((int64_t)blockIdx.x * EW_THREADS + threadIdx.x) * EW_PER_THREAD; i < n; i += stride) {
        uint32_t w = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (i + t < n) w |= (uint32_t)q[i + t] << (8 * t);
        if constexpr (ODT == TFP8_F32) {
            float v[4];
            dec4_f32<FMT>(w, v);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (i + t < n) ((float*)out)[i + t] = v[t];
        } else {
            const uint32_t p0 = ODT == TFP8_BF16 ? cvt2_bf16<FMT>(w, false) : cvt2_f16<FMT>(w, false);
            const uint32_t p1 = ODT == TFP8_BF16 ? cvt2_bf16<FMT>(w, true) : cvt2_f16<FMT>(w, true);
            const uint16_t h[4] = {(uint16_t)p0, (uint16_t)(p0 >> 16), (uint16_t)p1, (uint16_t)(p1 >> 16)};
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (i + t < n) ((uint16_t*)out)[i + t] = h[t];
        }
    }
}

// ------------------------------------------------------------------ encode
template <int FMT, int XDT>
__global__ __launch_bounds__(EW_THREADS) void encode_kernel(const void* __restrict__ x, int64_t n,
                                                            uint8_t* __restrict__ q) {
    const int64_t stride = (int64_t)gridDim.x * EW_THREADS * EW_PER_THREAD;
    for (int64_t i = ((int64_t)blockIdx.x * EW_THREADS + threadIdx.x) * EW_PER_THREAD; i < n; i += stride) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (i + t < n) q[i + t] = (uint8_t)encode_fp8<FMT>(load_elem<XDT>(x, i + t));
    }
}

// ------------------------------------------------------------------ quantize_weight
// One wave per (row n, K-group g), four groups per block: group amax (NaN propagates, as
// torch.amax does), scale s = max(amax/max_finite, FLT_MIN), the power-of-two ceiling of
// tfp8/quantize.py:11-12 when requested (pow2_ceil_ref: the rounding of torch's fp32 log2), s = 1
// for an all-zero group, then q = encode(w / s) (the encoder saturates, which equals
// clamp-then-RNE of tfp8/quantize.py:29-35).  UE8M0 stores log2 of that power of two + 127.
template <int FMT, int XDT, int SK>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w, int N, int K, int G,
                                                       int ng, int pow2, uint8_t* __restrict__ q,
                                                       void* __restrict__ scale) {
    const int64_t grp = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (grp >= (int64_t)N * ng) return;   // wave-uniform
    const int64_t n = grp / ng, g = grp % ng;
    const size_t base = (size_t)n * K + (size_t)g * G;
    float amax = 0.f;
    bool nan = false;
    for (int k = lane; k < G; k += 64) {
        const float v = load_elem<XDT>(w, base + k);
        nan |= __builtin_isnan(v);
        amax = fmaxf(amax, fabsf(v));
    }
    amax = wave_max(amax);
    const bool any_nan = __any(nan);
    float s;
    if (any_nan) {
        s = __uint_as_float(0x7FC00000u);
    } else {
        s = fmaxf(amax / Fmt<FMT>::MAX_FINITE, FLT_MIN);
        if (pow2 || SK == TFP8_SCALE_UE8M0) s = pow2_ceil_ref(s);
        if (amax == 0.f) s = 1.f;
    }
    for (int k = lane; k < G; k += 64) q[base + k] = (uint8_t)encode_fp8<FMT>(load_elem<XDT>(w, base + k) / s);
    if (lane == 0) {
        if constexpr (SK == TFP8_SCALE_UE8M0) {
            uint32_t e;
            if (any_nan) {
                e = 255u;
            } else {
                int ex = (int)((__float_as_uint(s) >> 23) & 0xFF) - 127;   // s is a normal power of two
                ex = ex < -127 ? -127 : (ex > 127 ? 127 : ex);
                e = (uint32_t)(ex + 127);
            }
            ((uint8_t*)scale)[grp] = (uint8_t)e;
        } else {
            ((float*)scale)[grp] = s;
        }
    }
}

// ------------------------------------------------------------------ prepare_activations
// One block per row.  e = ceil(log2(max(amax, 2^-100))) - 8 with the rounding of torch's fp32
// log2 (ceil_log2_ref), 0 when amax == 0 (tfp8/quantize.py:54-61); x16 = fp16(x * 2^-e), xs = 2^e.
template <int XDT>
__global__ __launch_bounds__(256) void prep_kernel(const void* __restrict__ x, int K,
                                                   uint16_t* __restrict__ x16, float* __restrict__ xs) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const size_t row = (size_t)m * K;
    float amax = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(load_elem<XDT>(x, row + k)));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (amax > 0.f) {
        e = ceil_log2_ref(fmaxf(amax, 0x1p-100f)) - 8;   // ACT_TARGET_EXP
    }
    const float inv = __uint_as_float((uint32_t)(127 - e) << 23);   // 2^-e, e in [-108, 121]
    for (int k = threadIdx.x; k < K; k += 256) x16[row + k] = f32_to_f16_bits(load_elem<XDT>(x, row + k) * inv);
    if (threadIdx.x == 0) xs[m] = __uint_as_float((uint32_t)(127 + e) << 23);
}

// ------------------------------------------------------------------ dequant
// out[n,k] = decode(w[n,k]) * scale(n, k/G), one f32 multiply then the output rounding, as in
// tfp8/quantize.py:39-44 (f32) and tfp8/csrc/tfp8_kernels.cu:435-456 (f16).
template <int FMT, int SK, int ODT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, int N, int K,
                                                      const void* __restrict__ ws, int G, int ng,
                                                      void* __restrict__ out) {
    const int64_t total = (int64_t)N * K;
    const int64_t stride = (int64_t)gridDim.x * 256 * 4;
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < total; i += stride) {
        uint32_t word = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (i + t < total) word |= (uint32_t)w[i + t] << (8 * t);
        float v[4];
        dec4_f32<FMT>(word, v);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t j = i + t;
            if (j < total) {
                const int64_t n = j / K, k = j % K;
                const float s = load_scale<SK>(ws, (size_t)n * ng + k / G);
                store_elem(out, j, ODT, v[t] * s);
            }
        }
    }
}

}  // namespace tfp8

using namespace tfp8;

extern "C" int tfp8_decode(const uint8_t* q, int64_t n, int fmt, void* out, int out_dtype, void* stream) {
    clear_error();
    if (n < 0 || !valid_fmt(fmt) || !valid_dtype(out_dtype))
        return fail(TFP8_ERR_ARG, "tfp8_decode: bad n/fmt/out_dtype (%lld, %d, %d)", (long long)n, fmt, out_dtype);
    if (n == 0) return 0;
    if (!q || !out) return fail(TFP8_ERR_ARG, "tfp8_decode: null pointer");
    const unsigned grid = grid_for(n, EW_THREADS * EW_PER_THREAD);
    hipStream_t s = (hipStream_t)stream;
    TFP8_DISPATCH_FMT(fmt, F, TFP8_DISPATCH_DT(out_dtype, D,
        decode_kernel<F, D><<<grid, EW_THREADS, 0, s>>>(q, n, out)));
    return check_launch("tfp8_decode");
}

extern "C" int tfp8_encode(const void* x, int x_dtype, int64_t n, int fmt, uint8_t* q, void* stream) {
    clear_error();
    if (n < 0 || !valid_fmt(fmt) || !valid_dtype(x_dtype))
        return fail(TFP8_ERR_ARG, "tfp8_encode: bad n/fmt/x_dtype (%lld, %d, %d)", (long long)n, fmt, x_dtype);
    if (n == 0) return 0;
    if (!q || !x) return fail(TFP8_ERR_ARG, "tfp8_encode: null pointer");
    const unsigned grid = grid_for(n, EW_THREADS * EW_PER_THREAD);
    hipStream_t s = (hipStream_t)stream;
    TFP8_DISPATCH_FMT(fmt, F, TFP8_DISPATCH_DT(x_dtype, D,
        encode_kernel<F, D><<<grid, EW_THREADS, 0, s>>>(x, n, q)));
    return check_launch("tfp8_encode");
}

extern "C" int tfp8_quantize_weight(const void* w, int w_dtype, int N, int K, int G, int fmt, int pow2,
                                    int scale_kind, uint8_t* q, void* scale, void* stream) {
    clear_error();
    if (N < 0 || K < 0 || G <= 0 || !valid_fmt(fmt) || !valid_dtype(w_dtype) || !valid_sk(scale_kind))
        return fail(TFP8_ERR_ARG, "tfp8_quantize_weight: bad N/K/G/fmt/dtype/scale_kind");
    if (K % G) return fail(TFP8_ERR_SHAPE, "tfp8_quantize_weight: K=%d not divisible by G=%d", K, G);
    if (N == 0 || K == 0) return 0;
    if (!w || !q || !scale) return fail(TFP8_ERR_ARG, "tfp8_quantize_weight: null pointer");
    const int ng = K / G;
    const int64_t groups = (int64_t)N * ng;
    const unsigned grid = (unsigned)((groups + 3) / 4);
    hipStream_t s = (hipStream_t)stream;
    TFP8_DISPATCH_FMT(fmt, F, TFP8_DISPATCH_DT(w_dtype, D, TFP8_DISPATCH_SK(scale_kind, S,
        quantize_kernel<F, D, S><<<grid, 256, 0, s>>>(w, N, K, G, ng, pow2, q, scale))));
    return check_launch("tfp8_quantize_weight");
}

extern "C" int tfp8_prepare_activations(const void* x, int x_dtype, int M, int K, void* x16, float* xs,
                                        void* stream) {
    clear_error();
    if (M < 0 || K < 0 || !valid_dtype(x_dtype))
        return fail(TFP8_ERR_ARG, "tfp8_prepare_activations: bad M/K/x_dtype");
    if (M == 0) return 0;
    if (!x || !x16 || !xs) return fail(TFP8_ERR_ARG, "tfp8_prepare_activations: null pointer");
    hipStream_t s = (hipStream_t)stream;
    TFP8_DISPATCH_DT(x_dtype, D, prep_kernel<D><<<M, 256, 0, s>>>(x, K, (uint16_t*)x16, xs));
    return check_launch("tfp8_prepare_activations");
}

extern "C" int tfp8_dequant(const uint8_t* w, int N, int K, const void* ws, int ws_kind, int G, int fmt,
                            void* out, int out_dtype, void* stream) {
    clear_error();
    if (N < 0 || K < 0 || G <= 0 || !valid_fmt(fmt) || !valid_dtype(out_dtype) || !valid_sk(ws_kind))
        return fail(TFP8_ERR_ARG, "tfp8_dequant: bad N/K/G/fmt/dtype/scale_kind");
    if (K % G) return fail(TFP8_ERR_SHAPE, "tfp8_dequant: K=%d not divisible by G=%d", K, G);
    if (N == 0 || K == 0) return 0;
    if (!w || !ws || !out) return fail(TFP8_ERR_ARG, "tfp8_dequant: null pointer");
    const unsigned grid = grid_for((int64_t)N * K, 256 * 4);
    hipStream_t s = (hipStream_t)stream;
    TFP8_DISPATCH_FMT(fmt, F, TFP8_DISPATCH_SK(ws_kind, S, TFP8_DISPATCH_DT(out_dtype, D,
        dequant_kernel<F, S, D><<<grid, 256, 0, s>>>(w, N, K, ws, G, K / G, out))));
    return check_launch("tfp8_dequant");
}
