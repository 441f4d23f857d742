// Shared device helpers and host plumbing for libtfp8_hip.so (gfx950 / CDNA4).
//
// Formula served by every kernel (the tfp8 W8A16 linear, reference tfp8/csrc/tfp8_kernels.cu:5-12):
//   y[m,n] = sum_k x[m,k] * decode(w[n,k]) * scale(n, k/G) + bias[n]        (fp32 accumulation)
// FP8 codes are uint8 (E4M3FN: 1-4-3 bias 7, no inf, NaN = S.1111.111, max 448;
// E5M2: 1-5-2 bias 15, IEEE inf/NaN, max 57344; tfp8/formats.py:30-31).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "tfp8_hip.h"

namespace tfp8 {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ host error plumbing
// Records a message for tfp8_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks the launch that was just issued; returns 0 or the hipError_t (with a message).
int check_launch(const char* what);
// Clears the thread's last-error message at the start of an entry point.
void clear_error();

// ------------------------------------------------------------------ tuning knobs (tuning.hip)
// Kernel-selection overrides, read from the environment once at library load and changed only
// through tfp8_tuning_set(); the launch path reads them with tune(), never with getenv.
enum Tune {
    TUNE_GEMV_CFG, TUNE_GEMV_WPC, TUNE_GEMV_MFMA_MIN, TUNE_GEMV_MFMA_MAX_M, TUNE_GM_NT, TUNE_GM_W, TUNE_GM_D,
    TUNE_GM_TL, TUNE_GEMM_TILE, TUNE_GEMM_SPLITK, TUNE_GEMM_DIRECT, TUNE_GEMM_DIRECT_MIN_M, TUNE_GEMM_DCFG,
    TUNE_GS_NW, TUNE_GS_KCS, TUNE_GS_SPLITK, TUNE_GS_TL, TUNE_GEMM_V1, TUNE_GEMV_PAIR, TUNE_GEMV_PAIR_MAX_M, TUNE_GEMV_QUAD, TUNE_GEMV_QUAD_MIN_M, TUNE_COUNT
};
int tune(Tune k);

// Returned by a kernel family's run_* function when it does not take the shape (the caller then
// tries the next family).  Distinct from 0, from every TFP8_ERR_* code and from every hipError_t.
constexpr int NOT_TAKEN = -1000;

// ------------------------------------------------------------------ format constants
template <int FMT> struct Fmt;
template <> struct Fmt<TFP8_E4M3FN> {
    static constexpr int MBITS = 3, BIAS = 7;
    static constexpr uint32_t MAX_BITS = 0x43E00000u;   // 448.0f
    static constexpr uint32_t MAX_CODE = 0x7Eu;
    static constexpr uint32_t NAN_CODE = 0x7Fu;         // tfp8/formats.py:94
    static constexpr float MAX_FINITE = 448.0f;
};
template <> struct Fmt<TFP8_E5M2> {
    static constexpr int MBITS = 2, BIAS = 15;
    static constexpr uint32_t MAX_BITS = 0x47600000u;   // 57344.0f
    static constexpr uint32_t MAX_CODE = 0x7Bu;
    static constexpr uint32_t NAN_CODE = 0x7Eu;         // tfp8/formats.py:94
    static constexpr float MAX_FINITE = 57344.0f;
};

// ------------------------------------------------------------------ decode (gfx950 cvt)
// gfx950 converts OCP FP8 in hardware: v_cvt_pk_f32_fp8 / _bf8 take the byte pair selected by
// `hi` (bytes 0,1 or 2,3 of the dword).  Every E4M3FN/E5M2 value is exact in f32, f16 and
// bf16, so the conversions below are exact for all 256 codes (checked on the device against
// the oracle for every code and byte position).
template <int FMT>
__device__ __forceinline__ f32x2 cvt2_f32(uint32_t w, bool hi) {
    if constexpr (FMT == TFP8_E4M3FN) return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true)
                                                : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
    else return hi ? __builtin_amdgcn_cvt_pk_f32_bf8(w, true) : __builtin_amdgcn_cvt_pk_f32_bf8(w, false);
}

// 4 codes of one dword -> 4 floats in byte order.
template <int FMT>
__device__ __forceinline__ void dec4_f32(uint32_t w, float* o) {
    f32x2 lo = cvt2_f32<FMT>(w, false), hi = cvt2_f32<FMT>(w, true);
    o[0] = lo.x; o[1] = lo.y; o[2] = hi.x; o[3] = hi.y;
}

// 2 codes -> packed bf16 / f16 pair (scale 1.0 is the identity for the scaled converts).
template <int FMT>
__device__ __forceinline__ uint32_t cvt2_bf16(uint32_t w, bool hi) {
    bf16x2 v;
    if constexpr (FMT == TFP8_E4M3FN)
        v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
               : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    else
        v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true)
               : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false);
    return __builtin_bit_cast(uint32_t, v);
}
template <int FMT>
__device__ __forceinline__ uint32_t cvt2_f16(uint32_t w, bool hi) {
    f16x2 v;
    if constexpr (FMT == TFP8_E4M3FN)
        v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true)
               : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
    else
        v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, true)
               : __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, false);
    return __builtin_bit_cast(uint32_t, v);
}

// ------------------------------------------------------------------ encode (exact RNE)
// f32 -> FP8 code, round-to-nearest-even on the bit pattern, saturating at +-max_finite
// (inf included), NaN -> the format's canonical NaN code with the sign dropped.  This is the
// rule of tfp8/formats.py:77-96 (nearest finite code, ties to the even code, clamp to max)
// computed arithmetically instead of by table search.
template <int FMT>
__device__ __forceinline__ uint32_t encode_fp8(float x) {
    using F = Fmt<FMT>;
    const uint32_t b = __float_as_uint(x);
    const uint32_t sign = (b >> 24) & 0x80u;
    const uint32_t a = b & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return F::NAN_CODE;
    if (a >= F::MAX_BITS) return sign | F::MAX_CODE;
    constexpr uint32_t MIN_NORMAL_BITS = (uint32_t)(127 + 1 - F::BIAS) << 23;
    if (a < MIN_NORMAL_BITS) {
        // Subnormal range: the code's mantissa is rne(|x| / 2^(1-bias-mbits)); a result of
        // 2^mbits is exactly the smallest normal code, which the same integer also encodes.
        const float t = __uint_as_float(a) * (float)(1u << (F::BIAS - 1 + F::MBITS));
        return sign | (uint32_t)__builtin_rintf(t);
    }
    constexpr int SH = 23 - F::MBITS;
    uint32_t r = a + ((1u << (SH - 1)) - 1u) + ((a >> SH) & 1u);
    r >>= SH;
    r -= (uint32_t)(127 - F::BIAS) << F::MBITS;
    return sign | r;
}

// ------------------------------------------------------------------ element I/O
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, size_t i) {
    if constexpr (DT == TFP8_F32) return ((const float*)p)[i];
    else if constexpr (DT == TFP8_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    else return f16_bits_to_f32(((const uint16_t*)p)[i]);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Runtime-dtype store (the branch is uniform across the launch).
__device__ __forceinline__ void store_elem(void* p, size_t i, int dt, float v) {
    if (dt == TFP8_F32) ((float*)p)[i] = v;
    else if (dt == TFP8_BF16) ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
    else ((uint16_t*)p)[i] = f32_to_f16_bits(v);
}

// ------------------------------------------------------------------ scales
// UE8M0 byte -> 2^(b-127); 255 is NaN (fp8_gemm_kernel.cu:22-30 rule), 0 is the subnormal 2^-127.
// Branch-free: e << 23 is the normal value (and 0x7F800000 for 255); e = 0 and e = 255 (the two
// bytes whose (e + 1) & 0xFF is at most 1) also set bit 22, giving 0x00400000 and 0x7FC00000.
__device__ __forceinline__ float ue8m0_to_f32(uint32_t e) {
    return __uint_as_float((e << 23) | (((e + 1u) & 0xFFu) <= 1u ? 0x00400000u : 0u));
}

template <int SK>
__device__ __forceinline__ float load_scale(const void* ws, size_t i) {
    if constexpr (SK == TFP8_SCALE_UE8M0) return ue8m0_to_f32(((const uint8_t*)ws)[i]);
    else return ((const float*)ws)[i];
}

// ceil(log2 s) exactly as a correctly rounded fp32 log2 followed by ceil computes it -- the
// formula torch.exp2(torch.ceil(torch.log2(s))) of tfp8/quantize.py:11-12 and :58-59 -- for a
// positive normal finite f32 s.  With s = 2^k (1 + j 2^-23), j > 0, the true log2 is
// k + log2(1 + j 2^-23); it rounds to exactly k, and the ceiling is then k instead of k + 1, when
// log2(1 + j 2^-23) is below half the gap from k to the next f32 value toward +inf.  That gap is
// 2^(floor(log2|k|) - 23), or half that for a negative k that is a power of two (the next value
// toward zero lies in the binade below).  Since log2(1 + f) = f / ln2 to within a relative 1e-5
// here, the condition is j <= floor(ln2 * 2^p) with p = floor(log2 gap) + 22, which is 0 for
// |k| < 4 and at most 22 (|k| >= 64).  Checked for every k and j <= 80 against torch's log2.
__device__ __forceinline__ int ceil_log2_ref(float s) {
    const uint32_t b = __float_as_uint(s);
    const int k = (int)((b >> 23) & 0xFF) - 127;
    const uint32_t j = b & 0x007FFFFFu;
    if (j == 0u) return k;
    if (k == 0) return 1;
    const int ak = k < 0 ? -k : k;
    int fl = 31 - __builtin_clz((unsigned)ak);        // floor(log2 |k|), 0..6
    if (k < 0 && (ak & (ak - 1)) == 0) fl -= 1;
    // floor(ln2 * 2^p) for p = fl - 1 = -2 .. 5
    constexpr uint32_t JMAX[8] = {0u, 0u, 0u, 1u, 2u, 5u, 11u, 22u};
    return j <= JMAX[fl + 1] ? k : k + 1;
}

// 2^ceil(log2 s) with the rounding of ceil_log2_ref (inf and NaN pass through; s positive and
// normal otherwise, as every caller clamps it to >= FLT_MIN first).
__device__ __forceinline__ float pow2_ceil_ref(float s) {
    const uint32_t b = __float_as_uint(s);
    if ((b & 0x7F800000u) == 0x7F800000u) return s;
    const int e = ceil_log2_ref(s);
    return e > 127 ? __uint_as_float(0x7F800000u) : __uint_as_float((uint32_t)(e + 127) << 23);
}

// ------------------------------------------------------------------ wave reductions (DPP)
// Sum over the 16 lanes of a DPP row; every lane of the row ends with the total.
//   quad_perm [1,0,3,2] and [2,3,0,1] -> quad sums, row_half_mirror -> 8-lane sums,
//   row_mirror -> 16-lane sums.
#define TFP8_DPP(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, true))
__device__ __forceinline__ float row16_sum(float v) {
    v += TFP8_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
    v += TFP8_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
    v += TFP8_DPP(v, 0x141);  // row_half_mirror
    v += TFP8_DPP(v, 0x140);  // row_mirror
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, TFP8_DPP(v, 0xB1));
    v = fmaxf(v, TFP8_DPP(v, 0x4E));
    v = fmaxf(v, TFP8_DPP(v, 0x141));
    v = fmaxf(v, TFP8_DPP(v, 0x140));
    return v;
}
// Max over the whole 64-lane wave (all lanes must be active); result is wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Grid-stride helper for elementwise kernels: blocks of 256 threads, <= 8 waves/CU worth of work.
inline unsigned grid_for(int64_t items, int per_block) {
    int64_t g = (items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (unsigned)g;
}

inline bool valid_dtype(int d) { return d == TFP8_F16 || d == TFP8_BF16 || d == TFP8_F32; }
inline bool valid_fmt(int f) { return f == TFP8_E4M3FN || f == TFP8_E5M2; }
inline bool valid_sk(int s) { return s == TFP8_SCALE_F32 || s == TFP8_SCALE_UE8M0; }

}  // namespace tfp8

// Runtime enum -> compile-time constant dispatch (one instantiation per value).
#define TFP8_DISPATCH_FMT(fmt, F, ...)                          \
    do {                                                        \
        if ((fmt) == TFP8_E4M3FN) { constexpr int F = TFP8_E4M3FN; __VA_ARGS__; } \
        else { constexpr int F = TFP8_E5M2; __VA_ARGS__; }      \
    } while (0)
#define TFP8_DISPATCH_DT(dt, D, ...)                            \
    do {                                                        \
        if ((dt) == TFP8_F16) { constexpr int D = TFP8_F16; __VA_ARGS__; } \
        else if ((dt) == TFP8_BF16) { constexpr int D = TFP8_BF16; __VA_ARGS__; } \
        else { constexpr int D = TFP8_F32; __VA_ARGS__; }       \
    } while (0)
#define TFP8_DISPATCH_SK(sk, S, ...)                            \
    do {                                                        \
        if ((sk) == TFP8_SCALE_UE8M0) { constexpr int S = TFP8_SCALE_UE8M0; __VA_ARGS__; } \
        else { constexpr int S = TFP8_SCALE_F32; __VA_ARGS__; } \
    } while (0)
