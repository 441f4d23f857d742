// Decode-size products on the matrix cores: a few (up to 16) activation rows, f16/bf16 activations.
//
// y[m,n] = sum_k x[m,k] * decode(w[n,k]) * s(n, k/G) + bias[n]   (reference GEMV formula,
// tfp8/csrc/tfp8_kernels.cu:171-269, for the rows the reference sends to its GEMV; M <= 16 here)
//
// With more than one activation row the per-row dot products of the streaming GEMV re-read the
// activations from LDS once per row and spend one VALU op per 2 products; here one
// v_mfma_f32_16x16x32_{f16,bf16} takes 16 weight rows x 32 k against all (up to 16) activation
// rows, so the VALU only decodes (v_cvt_scalef32_pk_*, half rate, 2 codes per op).  Layout:
//   * a block owns NT x 16 weight rows and all of K; its W waves split K into contiguous ranges and
//     add their 16 x 16 fp32 results in LDS at the end -- no partial sums leave the block and no
//     second kernel runs; each wave covers all NT row tiles, so one activation fragment feeds NT
//     weight tiles (every load instruction costs the same address-unit time whether it brings
//     weights or activations, so fewer activation loads per weight byte is what matters);
//   * lane l handles weight row l & 15 and the 16-byte k slot l >> 4 of every 64-byte chunk; the low
//     and high 8 codes of those 16 bytes are the B operands of two MFMAs, and the activation
//     operands are the same k positions of activation row l & 15, loaded from L2 (two 16-byte loads
//     per chunk; rows past M read zeros).  The weights are not loaded in that layout (16 rows x 64
//     bytes per load streams ~15 % slower than 256 contiguous bytes per row): a group of 4 chunks
//     arrives as 4 loads of 4 rows x 256 bytes, goes through a wave-private LDS tile and is read
//     back as operands (when every wave's K range is whole groups; else the direct layout);
//   * D chunks per wave are in flight; every load is unconditional (out-of-range rows, chunks and
//     the k tail read zeros through the buffer resources);
//   * scales: per channel in the epilogue; K-group scales of the block's rows are staged in LDS
//     once (no scale loads in the loop): UE8M0 ride in the conversion's scale operand (it applies a
//     power of two exactly), f32 with G % 64 == 0 multiply each chunk's fp32 MFMA result;
//   * blocks are renumbered so that each XCD owns a contiguous run of weight rows (each line of y
//     is written from one L2).
#include <stdlib.h>

#include "tfp8_common.h"

namespace tfp8 {

namespace {

constexpr uint32_t GM_BUF_FLAGS = 0x00020000u;
constexpr uint32_t GM_OOB = 0x80000000u;
enum { SM_CHANNEL = 0, SM_UE8M0 = 1, SM_F32 = 2 };

template <typename T> struct GvOp;
template <> struct GvOp<_Float16> {
    typedef f16x8 V;
    static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, float s, bool hi) {
        f16x2 v;
        if constexpr (FMT == TFP8_E4M3FN) v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, false);
        else v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, false);
        return __builtin_bit_cast(uint32_t, v);
    }
};
template <> struct GvOp<__bf16> {
    typedef bf16x8 V;
    static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, float s, bool hi) {
        bf16x2 v;
        if constexpr (FMT == TFP8_E4M3FN) v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, false);
        else v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, false);
        return __builtin_bit_cast(uint32_t, v);
    }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gv_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, (int)GM_BUF_FLAGS);
}
__device__ __forceinline__ uint4 gv_load16(__amdgpu_buffer_rsrc_t r, uint32_t off, int aux) {
    return aux ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2))
               : __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Two 4-wave blocks per CU at least: the register cap this gives the compiler (C2 M=8 / C3 M=16:
// 14.84 -> 14.70 / 15.60 -> 15.10 us with the default configuration; 4 waves, 4 chunks in flight,
// 160 -> 152 VGPRs) also lets the 8-chunk form fit two waves per SIMD (308 -> 248 VGPRs).
template <typename T, int FMT, int SMODE, int NT, int W, int D, bool TL>
__global__ __launch_bounds__(64 * W, 512 / (64 * W)) void gemv_mfma_kernel(const T* __restrict__ x, const float* __restrict__ xs,
                                                           const uint8_t* __restrict__ w, const void* __restrict__ ws,
                                                           int sk, const float* __restrict__ bias,
                                                           void* __restrict__ y, int ydt, int M, int N, int K, int G,
                                                           int ng, int gshift, int sbytes, int rb) {
    using Op = GvOp<T>;
    typedef typename Op::V V;
    // rb weight rows per block: 16 NT, or 8 (one half-used tile: the other rows read zeros through
    // the weight resource and are not stored) to give a small N twice the blocks
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    f32x4* red = (f32x4*)(smem + sbytes);         // [W][NT][64] wave results
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, q = lane >> 4;

    const int nblk = gridDim.x, xcd = blockIdx.x & 7, q8 = nblk >> 3, r8 = nblk & 7;
    const int n0 = (xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3)) * rb;
    const int rows = min(rb, N - n0);

    const int cpr = (K + 63) >> 6;                // 64-byte chunks per row
    const int cw = (cpr + W - 1) / W;
    const int c0 = wave * cw, c1 = min(cpr, c0 + cw);
    const int nch = max(0, c1 - c0);

    const __amdgpu_buffer_rsrc_t wr = gv_rsrc(w + (size_t)n0 * K, (uint32_t)rows * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t xr = gv_rsrc(x, (uint32_t)M * (uint32_t)K * (uint32_t)sizeof(T));
    const uint32_t wlane = (uint32_t)j * (uint32_t)K + (uint32_t)q * 16u;
    const uint32_t xlane = ((uint32_t)j * (uint32_t)K + (uint32_t)q * 16u) * (uint32_t)sizeof(T);

    // Weight loads.  Direct layout (TL = false): load t of chunk c is the MFMA operand itself, 16 rows
    // x 64 bytes (lane l: row l & 15, 16 bytes at slot l >> 4).  Transposed layout (TL = true): the
    // 4 chunks of a 256-code group are 4 loads of 4 rows x 256 contiguous bytes each (lane l: row
    // 4a + (l >> 4), 16 bytes at l & 15), which stream from HBM ~15 % faster than 64-byte pieces of
    // 16 rows; the wave writes them to its own LDS tile and reads the operands back (LDS operations
    // of one wave complete in order, so no barrier).  TL processes D / 4 groups in flight.
    uint4 wb[D][NT], xa[D], xb[D];
    auto issue = [&](int d, int c) {
        const int k = c * 64 + q * 16;
        const bool ok = c < c1 && k < K;
        if constexpr (TL) {
            // d = 4 * group slot + a; c is the group's first chunk + a.  Load a of the group: rows
            // 4a .. 4a+3, bytes 64 * (c - a) .. +256 of each.
            const int a4 = d & 3, cg = c - a4;
            const int kk = cg * 64 + j * 16;
            const bool okg = cg < c1 && kk < K;
#pragma unroll
            for (int t = 0; t < NT; ++t)
                wb[d][t] = gv_load16(wr, okg ? (uint32_t)(t * 16 + 4 * a4 + q) * (uint32_t)K + (uint32_t)kk : GM_OOB, 1);
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                wb[d][t] = gv_load16(wr, ok ? wlane + (uint32_t)(t * 16) * (uint32_t)K + (uint32_t)c * 64u : GM_OOB, 1);
        }
        xa[d] = gv_load16(xr, ok ? xlane + (uint32_t)c * 64u * (uint32_t)sizeof(T) : GM_OOB, 0);
        xb[d] = gv_load16(xr, ok ? xlane + ((uint32_t)c * 64u + 8u) * (uint32_t)sizeof(T) : GM_OOB, 0);
    };
    // TL: this wave's transpose tiles, NT x [16 rows][256 bytes], 16-byte unit u of row r at u ^ r.
    uint8_t* tls = smem + sbytes + W * NT * 64 * sizeof(f32x4) + (size_t)wave * NT * 4096;

    // Weight and activation loads of the first D chunks go out before the scales are staged.
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, c0 + d);

    // K-group scales of the block's rows, once per block: f32 [rows][ng] or UE8M0 bytes [rows][ng].
    if constexpr (SMODE != SM_CHANNEL) {
        const int cnt = rows * ng;
        if constexpr (SMODE == SM_F32) {
            const float* src = (const float*)ws + (size_t)n0 * ng;
            for (int i = tid; i < cnt; i += 64 * W) ((float*)smem)[i] = src[i];
        } else {
            const uint8_t* src = (const uint8_t*)ws + (size_t)n0 * ng;
            for (int i = tid; i < cnt; i += 64 * W) smem[i] = src[i];
        }
    }
    __syncthreads();

    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int d, int c) {
        const int k = c * 64 + q * 16;
        const int g = min(gshift >= 0 ? (k >> gshift) : k / G, ng - 1);
        if constexpr (TL) {
            if ((d & 3) == 0) {
                // The group's 4 loads (rows 4a + q, 16-byte unit j) into this wave's tiles.
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const int r = 4 * a4 + q;
                        *(uint4*)(tls + t * 4096 + r * 256 + 16 * (j ^ r)) = wb[d + a4][t];
                    }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int srow = min(t * 16 + j, rows - 1);
            float s = 1.f;
            if constexpr (SMODE == SM_UE8M0) s = ue8m0_to_f32(smem[srow * ng + g]);
            // operand of chunk c: row j, 16-byte unit 4 (c mod 4) + q of the group
            const uint4 wv = TL ? *(const uint4*)(tls + t * 4096 + j * 256 + 16 * ((4 * (d & 3) + q) ^ j)) : wb[d][t];
            uint4 lo, hi;
            lo.x = Op::template cvt<FMT>(wv.x, s, false);
            lo.y = Op::template cvt<FMT>(wv.x, s, true);
            lo.z = Op::template cvt<FMT>(wv.y, s, false);
            lo.w = Op::template cvt<FMT>(wv.y, s, true);
            hi.x = Op::template cvt<FMT>(wv.z, s, false);
            hi.y = Op::template cvt<FMT>(wv.z, s, true);
            hi.z = Op::template cvt<FMT>(wv.w, s, false);
            hi.w = Op::template cvt<FMT>(wv.w, s, true);
            if constexpr (SMODE == SM_F32) {
                f32x4 p = Op::mma(__builtin_bit_cast(V, xa[d]), __builtin_bit_cast(V, lo), f32x4{0.f, 0.f, 0.f, 0.f});
                p = Op::mma(__builtin_bit_cast(V, xb[d]), __builtin_bit_cast(V, hi), p);
                const float sf = ((const float*)smem)[srow * ng + g];
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(p[r], sf, acc[t][r]);
            } else {
                acc[t] = Op::mma(__builtin_bit_cast(V, xa[d]), __builtin_bit_cast(V, lo), acc[t]);
                acc[t] = Op::mma(__builtin_bit_cast(V, xb[d]), __builtin_bit_cast(V, hi), acc[t]);
            }
        }
    };

    // Steady state (every chunk of the round computed, every chunk D later issued): no branches, so
    // the compiler's wait counts stay exact.  With the conditional form below in the loop, the merge
    // points made it wait for every load in flight, D chunks of prefetch notwithstanding.
    int i = 0;
    for (; i + 2 * D <= nch; i += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            compute(d, c0 + i + d);
            issue(d, c0 + i + d + D);
        }
    }
    for (; i < nch; i += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i + d < nch) compute(d, c0 + i + d);
            if (i + d + D < nch) issue(d, c0 + i + d + D);
        }
    }

    // Sum the W waves' K ranges.  MFMA output layout: lane l holds activation rows 4(l>>4)+r of
    // weight row l & 15 of each row tile.
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64 + lane] = acc[t];
    __syncthreads();
    // Wave v finishes row tile v (NT <= W).
    if (wave >= NT) return;
    const int t = wave;
    f32x4 tot = red[t * 64 + lane];
    for (int v = 1; v < W; ++v) {
        const f32x4 u = red[(v * NT + t) * 64 + lane];
        tot[0] += u[0]; tot[1] += u[1]; tot[2] += u[2]; tot[3] += u[3];
    }
    if (t * 16 + j >= rows) return;
    const int n = n0 + t * 16 + j;
    float cs = 1.f;
    if constexpr (SMODE == SM_CHANNEL)
        cs = sk == TFP8_SCALE_UE8M0 ? ue8m0_to_f32(((const uint8_t*)ws)[n]) : ((const float*)ws)[n];
    const float bv = bias ? bias[n] : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * q + r;
        if (m < M) {
            const float v = tot[r] * cs;
            store_elem(y, (size_t)m * N + n, ydt, xs ? fmaf(v, xs[m], bv) : v + bv);
        }
    }
}

template <typename T, int FMT, int SMODE, int NT, int W, int D>
static void gm_launch(const void* x, const float* xs, const uint8_t* w, const void* ws, int sk, const float* bias,
                      void* y, int ydt, int M, int N, int K, int G, int ng, int gshift, int sbytes, bool tl,
                      hipStream_t s) {
    // Below N = 4096 one 16-row tile per block would leave CUs idle: 8 rows per block instead
    // (N=2048, K=5632, the C5 down projection, M=5/8/16: 8.26/9.09/10.81 -> 7.14/8.03/9.75 us).
    const int rb = NT == 1 && N < 16 * 256 ? 8 : 16 * NT;
    const unsigned grid = (unsigned)((N + rb - 1) / rb);
    const size_t lds = (size_t)sbytes + (size_t)W * NT * 64 * sizeof(f32x4) + (tl ? (size_t)W * NT * 4096 : 0);
    if (tl) {
        if constexpr (D % 4 == 0)
            gemv_mfma_kernel<T, FMT, SMODE, NT, W, D, true><<<grid, 64 * W, lds, s>>>(
                (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, sbytes, rb);
    } else {
        gemv_mfma_kernel<T, FMT, SMODE, NT, W, D, false><<<grid, 64 * W, lds, s>>>(
            (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, sbytes, rb);
    }
}

template <typename T, int FMT, int SMODE>
static void gm_pick(int NT, int W, int D, const void* x, const float* xs, const uint8_t* w, const void* ws, int sk,
                    const float* bias, void* y, int ydt, int M, int N, int K, int G, int ng, int gshift, int sbytes,
                    bool tl, hipStream_t s) {
#define TFP8_GM_CFG(NT_, W_, D_)                                                                                   \
    if (NT == NT_ && W == W_ && D == D_) {                                                                       \
        gm_launch<T, FMT, SMODE, NT_, W_, D_>(x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, sbytes, tl, s); \
        return;                                                                                                  \
    }
    TFP8_GM_CFG(2, 8, 4) TFP8_GM_CFG(2, 8, 8) TFP8_GM_CFG(2, 4, 4) TFP8_GM_CFG(2, 4, 8)
    TFP8_GM_CFG(1, 8, 4) TFP8_GM_CFG(1, 8, 8) TFP8_GM_CFG(1, 4, 4) TFP8_GM_CFG(1, 4, 8)
    TFP8_GM_CFG(4, 4, 4) TFP8_GM_CFG(4, 8, 4) TFP8_GM_CFG(4, 4, 2) TFP8_GM_CFG(2, 4, 2)
#undef TFP8_GM_CFG
    gm_launch<T, FMT, SMODE, 2, 4, 4>(x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, sbytes, false, s);
}

}  // namespace

// Validated by the caller (K % 16, G % 16, K % G, 16-byte aligned x and w).  Returns NOT_TAKEN, launching
// nothing, where this kernel does not apply: fp32 activations, M outside 1..16, or f32 K-group
// scales whose groups are not whole 64-byte chunks.
int run_gemv_mfma(const void* x, int x_dtype, const float* xs, int M, int K, const uint8_t* w, int N, const void* ws,
                  int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    if (x_dtype == TFP8_F32 || M < 1 || M > 16) return NOT_TAKEN;
    const int ng = K / G;
    const int sm = ng == 1 ? SM_CHANNEL : ws_kind == TFP8_SCALE_UE8M0 ? SM_UE8M0 : SM_F32;
    if (sm == SM_F32 && G % 64) return NOT_TAKEN;
    const int gshift = (G & (G - 1)) == 0 ? __builtin_ctz((unsigned)G) : -1;
    // Config: two 16-row weight tiles per block, K split over 4 waves, 4 chunks in flight per wave
    // (sweep on MI355X at C2 M=4/8) while that gives a block per CU; below N = 8192 one tile per
    // block (twice the blocks), 8 waves, 8 chunks in flight (M=5/8/16, N=2048, K=5632, an LLM
    // down projection: 12.1/12.6/14.3 -> 8.2/9.0/10.8 us).  Knobs TFP8_GM_NT / _W / _D force them.
    const bool few = N < 16 * 2 * 256;
    const int NT = tune(TUNE_GM_NT) > 0 ? tune(TUNE_GM_NT) : few ? 1 : 2;
    const int W = tune(TUNE_GM_W) > 0 ? tune(TUNE_GM_W) : few ? 8 : 4;
    const int D = tune(TUNE_GM_D) > 0 ? tune(TUNE_GM_D) : few ? 8 : 4;
    const int sbytes = sm == SM_CHANNEL ? 0 : (16 * NT * ng * (sm == SM_F32 ? 4 : 1) + 15) / 16 * 16;
    // Transposed weight loads (C2 M=4: 18.1 -> 15.0 us, M=8: 19.4 -> 15.4 us; identical results)
    // need whole 256-code groups in every wave's K range; knob TFP8_GM_TL=0 keeps the direct layout.
    bool tl = tune(TUNE_GM_TL) != 0 && D % 4 == 0 && K % (256 * W) == 0;
    if (tl && sbytes + W * NT * (1024 + 4096) > 64 * 1024) tl = false;   // transpose tiles do not fit
    if (sbytes + W * NT * 1024 > 64 * 1024) return NOT_TAKEN;                      // scales of the block's rows
#define TFP8_GM_SM(T_, F_)                                                                                    \
    {                                                                                                         \
        if (sm == SM_CHANNEL) gm_pick<T_, F_, SM_CHANNEL>(NT, W, D, x, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, sbytes, tl, s); \
        else if (sm == SM_UE8M0) gm_pick<T_, F_, SM_UE8M0>(NT, W, D, x, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, sbytes, tl, s); \
        else gm_pick<T_, F_, SM_F32>(NT, W, D, x, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, gshift, sbytes, tl, s); \
    }
    if (x_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_GM_SM(__bf16, F));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_GM_SM(_Float16, F));
    }
#undef TFP8_GM_SM
    return check_launch("tfp8 decode MFMA GEMV");
}

}  // namespace tfp8
