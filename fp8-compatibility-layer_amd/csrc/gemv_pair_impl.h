#pragma once
// Decode GEMV for 1 <= M <= 4 activation rows (16-bit activations, K <= 1024 * CPR, K % 16 == 0): one
// wave per pair of weight rows, every load of the pair in flight at once, no LDS staging of the
// scales.  The kernel template and its launcher; gemv_pair.hip instantiates CPR = 2, 4, 8 and holds
// the routing, gemv_pair_k.hip the other chunk counts (compiled in parallel).
//
// y[m,n] = sum_g s(n, g) * sum_{k in g} x[m,k] * decode(w[n, k]) + bias[n]   (tfp8/csrc/tfp8_kernels.cu:171-269)
//
// Layout (gfx950, 64-wide waves):
//   * a block of WPB (4, or 8 at M = 1 when that makes one block per CU) waves owns WPB row pairs;
//     wave p streams rows 2p and 2p+1, each as CPR loads of 1 KB (buffer_load_dwordx4, lane l holds
//     bytes 16l..16l+15 of the chunk), all 2*CPR loads issued at the start -- the wave never waits
//     for a chunk before the next one is requested; when K is not a whole number of chunks the
//     lanes past K in the last chunk read out of range (zeros);
//   * x (M * K * 2 bytes) is staged in LDS once per block, rows 1024 * CPR elements apart with zeros
//     past K, the only block-wide barrier; the weight loads are issued before it, so it never
//     delays them;
//   * K-group scales (G = 16 L, L = 4, 8 or 16 lanes per group): the 16 codes of a lane lie in one
//     group; a row's scales are loaded once, spread one per lane (lane j*L + i holds group
//     i*(1024/G) + j), and broadcast inside each L-lane segment with ds_swizzle, so every chunk's
//     partial sum is scaled with one FMA (no LDS, no barrier);
//   * per-channel scale and bias are applied to the row totals;
//   * decode: v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8} (2 codes per instruction, shared by the M
//     activation rows), products with v_dot2_f32_{bf16,f16} (exact), fp32 accumulation.
// Blocks are renumbered so that each XCD owns one contiguous run of rows (y lines written from one
// L2).  Rows past N read out-of-range zeros and are not stored; activation rows past M read zeros.
#include "gemv_impl.h"

namespace tfp8 {

// Waves (row pairs) per block at M = 1 (gemv_pair.hip).
int pair_waves_per_block(int pairs);

namespace {

// The scale of chunk c's group for this lane: the row's scales are spread one per lane (lane
// j*L + i holds group i*(1024/G) + j), and lane l needs the one held by lane (l & ~(L-1)) | c.
// ds_swizzle in bitmask mode (source = ((lane & and_mask) | or_mask) within each 32 lanes)
// broadcasts it inside each L-lane segment.
template <int L, int C>
__device__ __forceinline__ uint32_t group_scale(uint32_t v) {
    static_assert(L <= 32 && C < L, "segments of at most 32 lanes");
    constexpr int PATTERN = (C << 5) | (0x1F & ~(L - 1));
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, PATTERN);
}

// MT activation rows (M = MT, or M < MT with the rows past M reading zeros and not stored).
// Scale and bias loads are unconditional (a missing value reads out of range as zero): a load
// under a runtime branch made the compiler wait for it before issuing the weight loads.
// EXACT: K == 1024 * CPR, known at compile time (the C1 / C2 shapes: the run-time K arithmetic cost
// C1 ~0.06 us); otherwise K comes from k_arg and may end inside the last chunk.
template <int XDT, int FMT, int CPR, int L, bool UE8, int WPB, int MT, bool EXACT>
__global__ __launch_bounds__(64 * WPB) void gemv_pair_kernel(const void* __restrict__ x, const uint8_t* __restrict__ w,
                                                       const void* __restrict__ ws, const float* __restrict__ bias,
                                                       void* __restrict__ y, int ydt, int M, int N, int k_arg) {
    constexpr int KP = CPR * GEMV_CHUNK;                // x row stride in LDS (elements; zeros past K)
    const int K = EXACT ? KP : k_arg;
    constexpr bool GROUPED = L > 0;
    constexpr int TPB = 64 * WPB;
    constexpr int PPR = KP / 8;                         // 16-byte pieces of x per row
    constexpr int XN = MT * PPR;                        // 16-byte pieces of x
    constexpr int XQ = (XN + TPB - 1) / TPB;            // per thread
    static_assert(CPR <= 14 && XN * 16 <= 64 * 1024, "x of the block fits 64 KB of LDS");   // scales: CPR <= 14
    __shared__ uint4 xl[XN];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = gridDim.x, xcd = blockIdx.x & 7, q8 = nblk >> 3, r8 = nblk & 7;
    const int lb = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    const int n0 = (lb * WPB + wave) * 2;               // first row of this wave's pair

    // x first: its loads complete before any weight load, so waiting for them waits for nothing else.
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)(M * K * 2));
    uint4 xq[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {                      // piece p: row p / PPR, elements 8 (p % PPR) ..
        const int p = tid + q * TPB, m = p / PPR, kk = (p - m * PPR) * 8;
        if constexpr (EXACT) xq[q] = buf_load16(xr, (uint32_t)p * 16u, 0);                // past x: zeros
        else xq[q] = buf_load16(xr, kk < K ? (uint32_t)(m * K + kk) * 2u : BUF_OOB, 0);   // past x / K: zeros
    }

    // Scales and bias of the pair.  Grouped: lane j*L + i (i < CPR) loads group i*(1024/G) + j.
    const int ngk = GROUPED ? K / (16 * L) : 1;        // groups per row
    constexpr uint32_t SB = UE8 ? 1u : 4u;
    const __amdgpu_buffer_rsrc_t srs = buf_rsrc(ws, (uint32_t)N * (uint32_t)ngk * SB);
    int g = 0;
    bool gok = true;
    if constexpr (GROUPED) {                            // groups past K read zeros (the lanes using
        g = (lane % L) * (GEMV_CHUNK / (16 * L)) + lane / L;   // them multiply zero codes)
        gok = lane % L < CPR && g < ngk;
    }
    uint32_t sraw[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t off = gok && n0 + r < N ? ((uint32_t)(n0 + r) * (uint32_t)ngk + (uint32_t)g) * SB : BUF_OOB;
        if constexpr (UE8) sraw[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(srs, (int)off, 0, 0);
        else sraw[r] = __builtin_amdgcn_raw_buffer_load_b32(srs, (int)off, 0, 0);
    }
    const __amdgpu_buffer_rsrc_t brs = buf_rsrc(bias, bias ? (uint32_t)N * 4u : 0u);
    uint32_t braw[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
        braw[r] = __builtin_amdgcn_raw_buffer_load_b32(brs, n0 + r < N ? (n0 + r) * 4 : (int)BUF_OOB, 0, 0);

    // Every weight load of the pair.
    const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(w, (uint32_t)N * (uint32_t)K);
    const uint32_t lane16 = (uint32_t)lane * 16u;
    const uint32_t voff_last = EXACT || lane16 < (uint32_t)(K - (CPR - 1) * GEMV_CHUNK) ? lane16 : BUF_OOB;
    uint4 wv[CPR][2];
#pragma unroll
    for (int c = 0; c < CPR; ++c)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const bool ok = n0 + r < N;
            wv[c][r] = buf_load16<BUF_NT>(wrs, c == CPR - 1 ? voff_last : lane16,
                                          ok ? (uint32_t)(n0 + r) * (uint32_t)K + (uint32_t)(c * GEMV_CHUNK)
                                             : (uint32_t)N * (uint32_t)K);
        }

#pragma unroll
    for (int q = 0; q < XQ; ++q)
        if (XN % TPB == 0 || tid + q * TPB < XN) xl[tid + q * TPB] = xq[q];
    __syncthreads();

    // Each lane's scale for every chunk, as f32 (GROUPED), broadcast inside its L-lane segment.
    float sc[GROUPED ? CPR : 1][2];
    if constexpr (GROUPED) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const float f = UE8 ? ue8m0_to_f32(sraw[r]) : __uint_as_float(sraw[r]);
            const uint32_t fb = __float_as_uint(f);
            sc[0][r] = __uint_as_float(group_scale<L, 0>(fb));
            if constexpr (CPR > 1) sc[1][r] = __uint_as_float(group_scale<L, 1>(fb));
            if constexpr (CPR > 2) sc[2][r] = __uint_as_float(group_scale<L, 2>(fb));
            if constexpr (CPR > 3) sc[3][r] = __uint_as_float(group_scale<L, 3>(fb));
            if constexpr (CPR > 4) sc[4][r] = __uint_as_float(group_scale<L, 4>(fb));
            if constexpr (CPR > 5) sc[5][r] = __uint_as_float(group_scale<L, 5>(fb));
            if constexpr (CPR > 6) sc[6][r] = __uint_as_float(group_scale<L, 6>(fb));
            if constexpr (CPR > 7) sc[7][r] = __uint_as_float(group_scale<L, 7>(fb));
            if constexpr (CPR > 8) sc[8][r] = __uint_as_float(group_scale<L, 8>(fb));
            if constexpr (CPR > 9) sc[9][r] = __uint_as_float(group_scale<L, 9>(fb));
            if constexpr (CPR > 10) sc[10][r] = __uint_as_float(group_scale<L, 10>(fb));
            if constexpr (CPR > 11) sc[11][r] = __uint_as_float(group_scale<L, 11>(fb));
            if constexpr (CPR > 12) sc[12][r] = __uint_as_float(group_scale<L, 12>(fb));
            if constexpr (CPR > 13) sc[13][r] = __uint_as_float(group_scale<L, 13>(fb));
        }
    }

    float acc[MT][2];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m][0] = acc[m][1] = 0.f;
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
        uint32_t wk[2][8];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t d[4] = {wv[c][r].x, wv[c][r].y, wv[c][r].z, wv[c][r].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wk[r][2 * q] = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[q], false) : cvt2_f16<FMT>(d[q], false);
                wk[r][2 * q + 1] = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[q], true) : cvt2_f16<FMT>(d[q], true);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int xo = (m * KP + c * GEMV_CHUNK + lane * 16) / 8;
            const uint4 xa = xl[xo], xb = xl[xo + 1];
            const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float a = 0.f;
#pragma unroll
                for (int q = 0; q < 8; ++q) a = dot2_acc(xv[q], wk[r][q], a, XDT);
                if constexpr (GROUPED) acc[m][r] = fmaf(a, sc[c][r], acc[m][r]);
                else acc[m][r] += a;
            }
        }
    }

    float cs[2] = {1.f, 1.f};
    if constexpr (!GROUPED) {
#pragma unroll
        for (int r = 0; r < 2; ++r) cs[r] = UE8 ? ue8m0_to_f32(sraw[r]) : __uint_as_float(sraw[r]);
    }
    float out[MT][2];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 2; ++r) out[m][r] = wave_sum(acc[m][r]) * cs[r] + __uint_as_float(braw[r]);
    // Lane m stores row m's pair.
    float o0 = out[0][0], o1 = out[0][1];
#pragma unroll
    for (int m = 1; m < MT; ++m) {
        o0 = lane == m ? out[m][0] : o0;
        o1 = lane == m ? out[m][1] : o1;
    }
    if (lane < min(M, MT)) {
        const size_t o = (size_t)lane * N + n0;
        if (n0 + 1 < N && ydt != TFP8_F32) {
            const uint32_t h0 = ydt == TFP8_BF16 ? f32_to_bf16_bits(o0) : f32_to_f16_bits(o0);
            const uint32_t h1 = ydt == TFP8_BF16 ? f32_to_bf16_bits(o1) : f32_to_f16_bits(o1);
            *(uint32_t*)((uint16_t*)y + o) = h0 | (h1 << 16);
        } else if (n0 + 1 < N) {
            *(float2*)((float*)y + o) = make_float2(o0, o1);
        } else if (n0 < N) {
            store_elem(y, o, ydt, o0);
        }
    }
}

// Waves (row pairs) per block: 8 when a grid of 8-wave blocks is one block per CU (7/8 of the CUs
// or more busy), else 4.  Measured on MI355X (256 CUs), us per launch: C1 (2048 pairs) 8 per block
// 4.36, 4 per block 4.63; C2 M=1 (7168 pairs) 4 per block 10.56, 8 per block 10.92; 7, 14 or 16 per
// block were slower for both (5.3-5.9 and 11.1-12.1).

template <int XDT, int FMT, int CPR, int MT, bool EXACT>
void launch_pair_l(int L, bool ue8, const void* x, const uint8_t* w, const void* ws, const float* bias, void* y,
                   int ydt, int M, int N, int K, hipStream_t s) {
    const int pairs = (N + 1) / 2;
    const int wpb = MT == 1 ? pair_waves_per_block(pairs) : 4;
    const unsigned grid = (unsigned)((pairs + wpb - 1) / wpb);
#define TFP8_PAIR_W(LV, U, W) \
    gemv_pair_kernel<XDT, FMT, CPR, LV, U, W, MT, EXACT><<<grid, 64 * W, 0, s>>>(x, w, ws, bias, y, ydt, M, N, K)
#define TFP8_PAIR_U(LV, W) { if (ue8) TFP8_PAIR_W(LV, true, W); else TFP8_PAIR_W(LV, false, W); }
#define TFP8_PAIR(LV)                                         \
    {                                                         \
        if (MT == 1 && wpb == 8) TFP8_PAIR_U(LV, (MT == 1 ? 8 : 4)) \
        else TFP8_PAIR_U(LV, 4)                               \
    }
    if (L == 0) TFP8_PAIR(0)
    else if (L == 4) {
        if constexpr (CPR <= 4) TFP8_PAIR(4)   // the caller only passes L >= CPR
    } else if (L == 8) {
        if constexpr (CPR <= 8) TFP8_PAIR(8)
    } else TFP8_PAIR(16)
#undef TFP8_PAIR
#undef TFP8_PAIR_U
#undef TFP8_PAIR_W
}

}  // namespace

}  // namespace tfp8
