// Decode GEMV on the 4x4x4 matrix cores for a few (up to 8) activation rows, 16-bit activations,
// K = 2048 or 4096: one wave per four weight rows.
//
// y[m,n] = sum_g s(n, g) * sum_{k in g} x[m,k] * decode(w[n, k]) + bias[n]   (tfp8/csrc/tfp8_kernels.cu:171-269)
//
// v_mfma_f32_4x4x4_16b_{f16,bf16} runs 16 independent 4x4x4 products: in block b (lanes 4b..4b+3)
// lane i supplies row i of A and column i of B (4 k values each) and receives column i of the
// 4 x 4 result, D[m][i] for m = 0..3 (lane layout measured on the box).  Layout:
//   * wave p owns weight rows 4p .. 4p+3; lane (b = lane >> 2, i = lane & 3) loads the 16 codes
//     k = 256c + 16b .. +15 of row 4p + i for chunk c -- one buffer_load_dwordx4 moves 4 rows x 256
//     contiguous bytes -- and every chunk of the wave is requested at the start;
//   * the lane's 16 codes are the B columns of 4 MFMAs (4 k each); their A rows are the same 16 k
//     of activation row i (row i + 4 for the second set when M > 4), read from x staged in LDS once
//     per block.  Block b thus accumulates, for every (activation row, weight row) pair, the
//     products of its own k range, and the 16 blocks are added across lanes at the end;
//   * the products are exact (FP8 values and 16-bit activations), the sums fp32.  The VALU only
//     decodes (v_cvt_scalef32_pk_*, 8 per 16 codes); a dot-product GEMV spends 8 more VALU ops per
//     activation row, and the 4x4x4 MFMAs take about as long as 2 VALU ops each;
//   * K-group scales (G = 64, 128 or 256): the lane's 16 codes lie in one group, so each chunk's 4
//     MFMAs start from zero and their result is scaled with one fma per value.  The four rows' group
//     scales are loaded once (lane (b, i) holds groups GPC b .. GPC b + GPC - 1 of row 4p + i, GPC =
//     256 / G groups per chunk) and fetched for chunk c from lane 4c + i with ds_bpermute;
//   * one scale per row and the bias are applied to the totals.
// x is staged in LDS with 16-byte pieces XOR-swizzled per row (piece p of row r at p ^ f(r & 3),
// f = 0, 1, 8, 9): the 16 lanes of a quarter-wave read 16 distinct bank groups.
// Blocks are renumbered so that each XCD owns one contiguous run of rows.  Rows past N read
// out-of-range zeros and are not stored; activation rows past M read zeros.
#include "gemv_impl.h"

namespace tfp8 {

namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

template <int XDT>
__device__ __forceinline__ f32x4 mfma4(uint2 a, uint2 b, f32x4 c) {
    if constexpr (XDT == TFP8_BF16)
        return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

// Sum over the 16 lanes that share lane & 3 (lane, lane ^ 4, ..., lane ^ 60); every lane gets it.
__device__ __forceinline__ float quad_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (4 << 10) | 0x1F));
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (8 << 10) | 0x1F));
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (16 << 10) | 0x1F));
    const int l = (int)(__lane_id() ^ 32);
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(l << 2, __builtin_bit_cast(int, v)));
    return v;
}

__device__ __forceinline__ int quad_swz(int i) { return (i & 1) | ((i & 2) << 2); }

// NCH chunks of 256 codes per row (K = 256 NCH), GPC groups per chunk (0: one scale per row), MS
// sets of 4 activation rows; KS waves share a quad of rows, each taking NCH / KS chunks, and add
// their totals through LDS (a wave's chunks are processed one after another once they arrive, so
// fewer chunks per wave shorten the tail after the last data).
template <int XDT, int FMT, int NCH, int GPC, bool UE8, int WPB, int MS, int KS>
__global__ __launch_bounds__(64 * WPB) void gemv_quad_kernel(const void* __restrict__ x, const uint8_t* __restrict__ w,
                                                       const void* __restrict__ ws, const float* __restrict__ bias,
                                                       void* __restrict__ y, int ydt, int M, int N) {
    constexpr int K = NCH * 256;
    constexpr int TPB = 64 * WPB;
    constexpr int XR = 4 * MS;                           // activation rows in LDS
    constexpr int XN = XR * K / 8;                       // 16-byte pieces of x
    constexpr int XQ = (XN + TPB - 1) / TPB;             // per thread
    constexpr int CPW = NCH / KS;                        // chunks per wave
    static_assert(WPB % KS == 0 && CPW % 2 == 0, "whole chunk pairs per wave");
    static_assert(NCH <= 16 && NCH % 2 == 0 && (GPC == 0 || GPC == 1 || GPC == 2 || GPC == 4), "one chunk per lane block, G = 64 / 128 / 256");
    __shared__ uint4 xl[XN];
    const int tid = threadIdx.x, lane = tid & 63, qb = lane >> 2, qi = lane & 3;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = gridDim.x, xcd = blockIdx.x & 7, q8 = nblk >> 3, r8 = nblk & 7;
    const int lb = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    const int kh = wave % KS;                            // this wave's share of K
    const int n0 = (lb * (WPB / KS) + wave / KS) * 4;    // first row of this wave's four
    const int row = n0 + qi;                             // this lane's weight row

    // x first: its loads complete before any weight load, so waiting for them waits for nothing else.
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)(M * K * 2));
    uint4 xq[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) xq[q] = buf_load16(xr, (uint32_t)(tid + q * TPB) * 16u, 0);   // past x: zeros

    // Scales: grouped, lane (b, i) holds groups GPC b .. GPC b + GPC - 1 of its row; else the row's one.
    constexpr int NGK = GPC ? NCH * GPC : 1;             // groups per row
    constexpr int NPRE = GPC ? GPC : 1;
    constexpr uint32_t SB = UE8 ? 1u : 4u;
    const __amdgpu_buffer_rsrc_t srs = buf_rsrc(ws, (uint32_t)N * NGK * SB);
    uint32_t sraw[NPRE];
#pragma unroll
    for (int e = 0; e < NPRE; ++e) {
        const int g = GPC ? qb * GPC + e : 0;
        const uint32_t off = row < N && (!GPC || qb < NCH) ? ((uint32_t)row * NGK + (uint32_t)g) * SB : BUF_OOB;
        if constexpr (UE8) sraw[e] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(srs, (int)off, 0, 0);
        else sraw[e] = __builtin_amdgcn_raw_buffer_load_b32(srs, (int)off, 0, 0);
    }
    const __amdgpu_buffer_rsrc_t brs = buf_rsrc(bias, bias ? (uint32_t)N * 4u : 0u);
    const uint32_t braw = __builtin_amdgcn_raw_buffer_load_b32(brs, row < N ? row * 4 : (int)BUF_OOB, 0, 0);

    // Every weight load of the wave: chunk c = codes 256c + 16b .. +15 of the lane's row.
    const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(w, (uint32_t)N * (uint32_t)K);
    const uint32_t voff = row < N ? (uint32_t)row * (uint32_t)K + (uint32_t)qb * 16u : BUF_OOB;
    uint4 wv[CPW];
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) wv[cc] = buf_load16<BUF_NT>(wrs, voff, (uint32_t)((kh * CPW + cc) * 256));

#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const int piece = tid + q * TPB;
        if (XN % TPB == 0 || piece < XN) {
            const int r = piece / (K / 8), p = piece % (K / 8);
            xl[r * (K / 8) + (p ^ quad_swz(r & 3))] = xq[q];
        }
    }
    __syncthreads();

    float scf[NPRE];
#pragma unroll
    for (int e = 0; e < NPRE; ++e) scf[e] = UE8 ? ue8m0_to_f32(sraw[e]) : __uint_as_float(sraw[e]);

    // Two chunks per iteration, their MFMA chains interleaved (one chain's latency hides under the
    // other's issue): acc[s][0] takes even chunks, acc[s][1] odd ones (one scale per row).
    // Every chunk's group scale, fetched before the chunk loop (so the cross-lane fetches' latency
    // hides under the first chunks' work): group (256c + 16b) / G of the lane's row is held by lane
    // 4c + i at index b GPC / 16.
    float scl[GPC > 0 ? CPW : 1];
    if constexpr (GPC > 0) {
#pragma unroll
        for (int cc = 0; cc < CPW; ++cc) {
            const int src = (4 * (kh * CPW + cc) + qi) << 2;
            float v[GPC];
#pragma unroll
            for (int e = 0; e < GPC; ++e)
                v[e] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, scf[e])));
            scl[cc] = v[0];
            if constexpr (GPC == 2) scl[cc] = qb >= 8 ? v[1] : v[0];
            if constexpr (GPC == 4) {
                const int e = qb >> 2;
                scl[cc] = e == 0 ? v[0] : e == 1 ? v[1] : e == 2 ? v[2] : v[3];
            }
        }
    }
    f32x4 acc[MS][2];
#pragma unroll
    for (int s = 0; s < MS; ++s) acc[s][0] = acc[s][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int sw = quad_swz(qi);
#pragma unroll
    for (int cc0 = 0; cc0 < CPW; cc0 += 2) {
        const int c0 = kh * CPW + cc0;
        // B columns: 4 codes per MFMA, decoded exactly to the activation type.
        uint2 bq[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t d[4] = {wv[cc0 + h].x, wv[cc0 + h].y, wv[cc0 + h].z, wv[cc0 + h].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[j], false) : cvt2_f16<FMT>(d[j], false);
                const uint32_t hi = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[j], true) : cvt2_f16<FMT>(d[j], true);
                bq[h][j] = make_uint2(lo, hi);
            }
        }
#pragma unroll
        for (int s = 0; s < MS; ++s) {
            const int xbase = (qi + 4 * s) * (K / 8);
            uint2 a[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int p0 = 32 * (c0 + h) + 2 * qb;
                const uint4 xa = xl[xbase + (p0 ^ sw)], xb = xl[xbase + ((p0 + 1) ^ sw)];
                a[h][0] = make_uint2(xa.x, xa.y);
                a[h][1] = make_uint2(xa.z, xa.w);
                a[h][2] = make_uint2(xb.x, xb.y);
                a[h][3] = make_uint2(xb.z, xb.w);
            }
            if constexpr (GPC > 0) {
                f32x4 p[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int h = 0; h < 2; ++h) p[h] = mfma4<XDT>(a[h][j], bq[h][j], p[h]);
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[s][0][v] = fmaf(p[h][v], scl[GPC > 0 ? cc0 + h : 0], acc[s][0][v]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int h = 0; h < 2; ++h) acc[s][h] = mfma4<XDT>(a[h][j], bq[h][j], acc[s][h]);
            }
        }
        // one chunk pair at a time: hoisting every chunk's LDS reads and scale fetches to the top
        // costs more registers than the latency it hides
        __builtin_amdgcn_sched_barrier(0);
    }

    // Totals: lane i (b = 0) holds y[m + 4s][n0 + i] for m = 0..3 (this wave's share of K).
    float tot[MS][4];
#pragma unroll
    for (int s = 0; s < MS; ++s)
#pragma unroll
        for (int v = 0; v < 4; ++v) tot[s][v] = quad_sum(acc[s][0][v] + acc[s][1][v]);
    if constexpr (KS > 1) {
        __shared__ float red[WPB / KS][KS - 1][MS * 16];
        if (kh > 0 && qb == 0) {
#pragma unroll
            for (int s = 0; s < MS; ++s)
#pragma unroll
                for (int v = 0; v < 4; ++v) red[wave / KS][kh - 1][(s * 4 + v) * 4 + qi] = tot[s][v];
        }
        __syncthreads();
        if (kh > 0) return;
#pragma unroll
        for (int u = 0; u < KS - 1; ++u)
#pragma unroll
            for (int s = 0; s < MS; ++s)
#pragma unroll
                for (int v = 0; v < 4; ++v) tot[s][v] += red[wave / KS][u][(s * 4 + v) * 4 + qi];
    }
    const float cs = GPC ? 1.f : scf[0];
    const float bv = __uint_as_float(braw);
#pragma unroll
    for (int s = 0; s < MS; ++s)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = v + 4 * s;
            if (qb == 0 && m < M && row < N) store_elem(y, (size_t)m * N + row, ydt, tot[s][v] * cs + bv);
        }
}

template <int XDT, int FMT, int NCH, int MS>
void launch_quad(int gpc, bool ue8, const void* x, const uint8_t* w, const void* ws, const float* bias, void* y,
                 int ydt, int M, int N, hipStream_t s) {
    constexpr int KS = 2, WPB = 4 * KS;                  // 4 row quads per block
    const int quads = (N + 3) / 4;
    const unsigned grid = (unsigned)((quads + WPB / KS - 1) / (WPB / KS));
#define TFP8_QUAD(G_)                                                                                        \
    {                                                                                                        \
        if (ue8) gemv_quad_kernel<XDT, FMT, NCH, G_, true, WPB, MS, KS><<<grid, 64 * WPB, 0, s>>>(x, w, ws, bias, y, ydt, M, N); \
        else gemv_quad_kernel<XDT, FMT, NCH, G_, false, WPB, MS, KS><<<grid, 64 * WPB, 0, s>>>(x, w, ws, bias, y, ydt, M, N); \
    }
    if (gpc == 0) TFP8_QUAD(0)
    else if (gpc == 1) TFP8_QUAD(1)
    else if (gpc == 2) TFP8_QUAD(2)
    else TFP8_QUAD(4)
#undef TFP8_QUAD
}

}  // namespace

// Runs the 4x4x4-MFMA GEMV if it takes the shape; returns NOT_TAKEN otherwise.  It takes
// TFP8_GEMV_QUAD_MIN_M (default 3) <= M <= 8 rows of f16/bf16 activations with K = 2048 or 4096 and
// weights below 2^31 bytes, with one scale per row (knob TFP8_GEMV_QUAD = 1, the default) or also
// K-groups of 64/128/256 (TFP8_GEMV_QUAD = 2).  Measured on MI355X (us, this kernel vs the row-pair
// GEMV up to M = 4 and the matrix-core decode kernel above): one scale per row, N = K = 4096: M=2
// 5.09 vs 5.12, M=4 5.36 vs 5.75, M=8 6.57 vs 8.43; 128-groups, N = 14336, K = 4096: M=2 12.41 vs
// 11.39, M=4 13.44 vs 13.78, M=8 17.64 vs 14.83 -- with K-group scales each chunk's sums take a
// multiply-add per value and the group scale a cross-lane fetch, and the kernel loses above M = 4.
int run_gemv_quad(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                  int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    const int mode = tune(TUNE_GEMV_QUAD);
    if (mode <= 0 || M < tune(TUNE_GEMV_QUAD_MIN_M) || M < 1 || M > 8 || x_dtype == TFP8_F32) return NOT_TAKEN;
    if ((K != 2048 && K != 4096) || (long)N * K >= (1L << 31)) return NOT_TAKEN;
    int gpc = 0;
    if (G != K) {
        // K-group scales: from 3 to 4 rows by default (C2 M=3/4, G=128: 13.11 -> 12.88 / 13.83 -> 13.48
        // us against the row-pair GEMV), above that only when forced (M=8: 17.7 vs 14.8 us on the
        // matrix-core decode kernel).
        if ((mode < 2 && M > 4) || (G != 64 && G != 128 && G != 256)) return NOT_TAKEN;
        gpc = 256 / G;
    }
    const bool ue8 = ws_kind == TFP8_SCALE_UE8M0;
#define TFP8_QUAD_K(XD, F, MS)                                                                           \
    {                                                                                                   \
        if (K == 2048) launch_quad<XD, F, 8, MS>(gpc, ue8, x, w, ws, bias, y, y_dtype, M, N, s);        \
        else launch_quad<XD, F, 16, MS>(gpc, ue8, x, w, ws, bias, y, y_dtype, M, N, s);                 \
    }
#define TFP8_QUAD_M(XD, F)                      \
    {                                          \
        if (M <= 4) TFP8_QUAD_K(XD, F, 1)      \
        else TFP8_QUAD_K(XD, F, 2)             \
    }
    if (x_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_QUAD_M(TFP8_BF16, F));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_QUAD_M(TFP8_F16, F));
    }
#undef TFP8_QUAD_M
#undef TFP8_QUAD_K
    return check_launch("tfp8_gemv (quad)");
}

}  // namespace tfp8
