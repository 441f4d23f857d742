// Single-row decode GEMV (M = 1, 16-bit activations, K = 1024 * CPR): one wave per pair of
// weight rows, every load of the pair in flight at once, no LDS staging of the scales.
//
// y[n] = sum_g s(n, g) * sum_{k in g} x[k] * decode(w[n, k]) + bias[n]   (tfp8/csrc/tfp8_kernels.cu:171-269)
//
// Layout (gfx950, 64-wide waves):
//   * a block of WPB (4 or 8) waves owns WPB row pairs; wave p of the block streams rows 2p and
//     2p+1, each as CPR loads of 1 KB (buffer_load_dwordx4, lane l holds bytes 16l..16l+15
//     of the chunk), all 2*CPR loads issued at the start -- the wave never waits for a chunk
//     before the next one is requested;
//   * x (K * 2 bytes) is staged in LDS once per block, the only block-wide barrier; the weight
//     loads are issued before it, so it never delays them;
//   * K-group scales (G = 16 L, L = 4, 8 or 16 lanes per group): the 16 codes of a lane lie in one
//     group, the L lanes of a group first add their partial sums with DPP, and then lane
//     j*L + i multiplies chunk i's sum of group segment j by its own scale, loaded once per row at
//     the start (one dword or byte per lane, no LDS, no barrier);
//   * per-channel scale and bias are applied to the wave's two row totals;
//   * decode: v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8} (2 codes per instruction), products with
//     v_dot2_f32_{bf16,f16} (exact), fp32 accumulation.
// Blocks are renumbered so that each XCD owns one contiguous run of rows (y lines written from one
// L2).  Rows past N read out-of-range zeros and are not stored.
#include "gemv_impl.h"

namespace tfp8 {

namespace {

template <int L>
__device__ __forceinline__ float group_sum(float v) {
    v += TFP8_DPP(v, 0xB1);                       // quad_perm [1,0,3,2]
    v += TFP8_DPP(v, 0x4E);                       // quad_perm [2,3,0,1]
    if constexpr (L >= 8) v += TFP8_DPP(v, 0x141);   // row_half_mirror
    if constexpr (L >= 16) v += TFP8_DPP(v, 0x140);  // row_mirror
    return v;
}

// Scale and bias loads are unconditional (a missing value reads out of range as zero): a load
// under a runtime branch made the compiler wait for it before issuing the weight loads.
template <int XDT, int FMT, int CPR, int L, bool UE8, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemv_pair_kernel(const void* __restrict__ x, const uint8_t* __restrict__ w,
                                                       const void* __restrict__ ws, const float* __restrict__ bias,
                                                       void* __restrict__ y, int ydt, int N) {
    constexpr int K = CPR * GEMV_CHUNK;
    constexpr bool GROUPED = L > 0;
    constexpr int TPB = 64 * WPB;
    constexpr int XN = K * 2 / 16;                      // 16-byte pieces of x
    constexpr int XQ = (XN + TPB - 1) / TPB;            // per thread
    __shared__ uint4 xl[XN];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = gridDim.x, xcd = blockIdx.x & 7, q8 = nblk >> 3, r8 = nblk & 7;
    const int lb = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    const int n0 = (lb * WPB + wave) * 2;               // first row of this wave's pair

    // x first: its loads complete before any weight load, so waiting for them waits for nothing else.
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)(K * 2));
    uint4 xq[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) xq[q] = buf_load16(xr, (uint32_t)(tid + q * TPB) * 16u, 0);   // past x: zeros

    // Scales and bias of the pair.  Grouped: lane j*L + i (i < CPR) takes group i*(1024/G) + j.
    constexpr int NGK = GROUPED ? K / (16 * L) : 1;    // groups per row
    constexpr uint32_t SB = UE8 ? 1u : 4u;
    const __amdgpu_buffer_rsrc_t srs = buf_rsrc(ws, (uint32_t)N * NGK * SB);
    int g = 0;
    bool gok = true;
    if constexpr (GROUPED) {
        g = (lane % L) * (GEMV_CHUNK / (16 * L)) + lane / L;
        gok = lane % L < CPR;
    }
    uint32_t sraw[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t off = gok && n0 + r < N ? ((uint32_t)(n0 + r) * NGK + (uint32_t)g) * SB : BUF_OOB;
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
    uint4 wv[CPR][2];
#pragma unroll
    for (int c = 0; c < CPR; ++c)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const bool ok = n0 + r < N;
            wv[c][r] = buf_load16<BUF_NT>(wrs, lane16, ok ? (uint32_t)(n0 + r) * K + (uint32_t)(c * GEMV_CHUNK)
                                                         : (uint32_t)N * (uint32_t)K);
        }

#pragma unroll
    for (int q = 0; q < XQ; ++q)
        if (XN % TPB == 0 || tid + q * TPB < XN) xl[tid + q * TPB] = xq[q];
    __syncthreads();

    float part[2] = {0.f, 0.f};                         // grouped: this lane's scaled product; else sum
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
        const uint4 xa = xl[(c * GEMV_CHUNK + lane * 16) / 8], xb = xl[(c * GEMV_CHUNK + lane * 16) / 8 + 1];
        const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t d[4] = {wv[c][r].x, wv[c][r].y, wv[c][r].z, wv[c][r].w};
            float a = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t lo = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[q], false) : cvt2_f16<FMT>(d[q], false);
                const uint32_t hi = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[q], true) : cvt2_f16<FMT>(d[q], true);
                a = dot2_acc(xv[2 * q], lo, a, XDT);
                a = dot2_acc(xv[2 * q + 1], hi, a, XDT);
            }
            if constexpr (GROUPED) {
                const float gs = group_sum<L>(a);      // group (chunk c, segment lane / L), in all L lanes
                part[r] = lane % L == c ? gs : part[r];
            } else {
                part[r] += a;
            }
        }
    }

    float out[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        float v = part[r];
        if constexpr (GROUPED) {
            const float sc = UE8 ? ue8m0_to_f32(sraw[r]) : __uint_as_float(sraw[r]);
            v = lane % L < CPR ? v * sc : 0.f;
        }
        float t = wave_sum(v);
        if constexpr (!GROUPED) t *= UE8 ? ue8m0_to_f32(sraw[r]) : __uint_as_float(sraw[r]);
        out[r] = t + __uint_as_float(braw[r]);
    }
    if (lane == 0) {
        if (n0 + 1 < N && ydt != TFP8_F32) {
            const uint32_t h0 = ydt == TFP8_BF16 ? f32_to_bf16_bits(out[0]) : f32_to_f16_bits(out[0]);
            const uint32_t h1 = ydt == TFP8_BF16 ? f32_to_bf16_bits(out[1]) : f32_to_f16_bits(out[1]);
            *(uint32_t*)((uint16_t*)y + n0) = h0 | (h1 << 16);
        } else if (n0 + 1 < N) {
            *(float2*)((float*)y + n0) = make_float2(out[0], out[1]);
        } else if (n0 < N) {
            store_elem(y, (size_t)n0, ydt, out[0]);
        }
    }
}

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

template <int XDT, int FMT, int CPR>
void launch_pair_l(int L, bool ue8, const void* x, const uint8_t* w, const void* ws, const float* bias, void* y,
                   int ydt, int N, hipStream_t s) {
    const int pairs = (N + 1) / 2;
    const int wpb = pair_waves_per_block(pairs);
    const unsigned grid = (unsigned)((pairs + wpb - 1) / wpb);
#define TFP8_PAIR_W(LV, U, W) gemv_pair_kernel<XDT, FMT, CPR, LV, U, W><<<grid, 64 * W, 0, s>>>(x, w, ws, bias, y, ydt, N)
#define TFP8_PAIR_U(LV, W) { if (ue8) TFP8_PAIR_W(LV, true, W); else TFP8_PAIR_W(LV, false, W); }
#define TFP8_PAIR(LV)                       \
    {                                       \
        if (wpb == 8) TFP8_PAIR_U(LV, 8)    \
        else TFP8_PAIR_U(LV, 4)             \
    }
    if (L == 0) TFP8_PAIR(0)
    else if (L == 4) TFP8_PAIR(4)
    else if (L == 8) TFP8_PAIR(8)
    else TFP8_PAIR(16)
#undef TFP8_PAIR
#undef TFP8_PAIR_U
#undef TFP8_PAIR_W
}

}  // namespace

// Runs the pair GEMV if it takes the shape (M = 1, f16/bf16 x, K = 2048, 4096 or 8192, one scale per
// row or K-groups of 64/128/256 that the chunks cover, weights below 2^31 bytes, y aligned for the
// pair store); returns NOT_TAKEN otherwise.
int run_gemv_pair(const void* x, int x_dtype, int M, int K, const uint8_t* w, int N, const void* ws, int ws_kind,
                  int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s) {
    if (M != 1 || x_dtype == TFP8_F32 || !tune(TUNE_GEMV_PAIR)) return NOT_TAKEN;
    const int cpr = K / GEMV_CHUNK;
    if (K % GEMV_CHUNK || (cpr != 2 && cpr != 4 && cpr != 8) || (long)N * K >= (1L << 31)) return NOT_TAKEN;
    int L = 0;
    if (G != K) {
        L = G / 16;
        if ((L != 4 && L != 8 && L != 16) || L < cpr) return NOT_TAKEN;
    }
    if ((uintptr_t)y % (y_dtype == TFP8_F32 ? 8 : 4)) return NOT_TAKEN;
    const bool ue8 = ws_kind == TFP8_SCALE_UE8M0;
#define TFP8_PAIR_CPR(XD, F)                                                                         \
    {                                                                                               \
        if (cpr == 2) launch_pair_l<XD, F, 2>(L, ue8, x, w, ws, bias, y, y_dtype, N, s);             \
        else if (cpr == 4) launch_pair_l<XD, F, 4>(L, ue8, x, w, ws, bias, y, y_dtype, N, s);        \
        else launch_pair_l<XD, F, 8>(L, ue8, x, w, ws, bias, y, y_dtype, N, s);                     \
    }
    if (x_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_PAIR_CPR(TFP8_BF16, F));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, TFP8_PAIR_CPR(TFP8_F16, F));
    }
#undef TFP8_PAIR_CPR
    return check_launch("tfp8_gemv (pair)");
}

}  // namespace tfp8
