// Weight-streaming MFMA GEMM (M > 8): the FP8 weight tile goes HBM -> registers -> MFMA B operand,
// the activation tile goes L2 -> LDS -> MFMA A operand.
//
// y[m,n] = xs[m] * sum_k x[m,k] * decode(w[n,k]) * s(n, k/G) + bias[n]   (fp32 accumulation)
// (reference gemm_w8a16, tfp8/csrc/tfp8_kernels.cu:271-411), laid out for CDNA4:
//   * a block is 4 waves over a 64*NW-row slice of W (each wave owns NW 16-row MFMA tiles) and all
//     M rows (TM 16-row MFMA tiles), and one K slice (split-K over gridDim.y when the tile grid is
//     too small for 256 CUs; fp32 partials then go to the caller's workspace);
//   * weights are read with buffer_load_dwordx4 (non-temporal): the MFMA B operand of lane l is 16
//     consecutive codes of row (l & 15) at k = 64c + 16(l >> 4), whose low/high 8 codes feed two
//     v_mfma_f32_16x16x32_{f16,bf16} (the activation operand reads the same permuted k order).
//     With 256-code chunks the loads are 4 rows x 256 contiguous bytes each (16 rows x 64 bytes per
//     instruction streams ~15 % slower) and each wave regroups them through its own LDS tile;
//     shorter chunks load the operand layout directly;
//     a whole chunk of KCS*64 k for all NW tiles is in flight while the previous chunk is consumed;
//   * codes are decoded in registers with v_cvt_scalef32_pk_{f16,bf16}_{fp8,bf8}; UE8M0 K-group
//     scales ride in that instruction's scale operand (it multiplies by the scale's power of two,
//     which a UE8M0 scale is), f32 K-group scales (G % 64 == 0) multiply fp32 per-step partials,
//     per-channel scales are applied in the epilogue;
//   * the activation chunk (TM*16 rows x KCS*64 k, zero-padded rows/columns) is double-buffered in
//     LDS (row stride padded by 16 B, conflict-free ds_read_b128), filled through registers one
//     chunk ahead; out-of-range weight rows/columns read zeros from the buffer resource.
#include <algorithm>
#include <atomic>

#include "tfp8_common.h"

namespace tfp8 {

namespace {

constexpr uint32_t GS_BUF_FLAGS = 0x00020000u;
constexpr int GS_NT = 2;

template <typename T> struct GsOp;
template <> struct GsOp<_Float16> {
    typedef f16x8 V;
    static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, float s, bool hi) {
        f16x2 v;
        if constexpr (FMT == TFP8_E4M3FN) v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, false);
        else v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, false);
        return __builtin_bit_cast(uint32_t, v);
    }
};
template <> struct GsOp<__bf16> {
    typedef bf16x8 V;
    static __device__ __forceinline__ f32x4 mma(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, float s, bool hi) {
        bf16x2 v;
        if constexpr (FMT == TFP8_E4M3FN) v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, false);
        else v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, false);
        return __builtin_bit_cast(uint32_t, v);
    }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gs_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, (int)GS_BUF_FLAGS);
}

enum { GM_CHANNEL = 0, GM_UE8M0 = 1, GM_F32 = 2 };

}  // namespace

template <typename T, int FMT, int TM, int NW, int KCS, int GMODE, bool TL>
__global__ __launch_bounds__(256) void gemm_stream_kernel(
    const T* __restrict__ x, const float* __restrict__ xs, const uint8_t* __restrict__ w, const void* __restrict__ ws,
    int sk, const float* __restrict__ bias, void* __restrict__ y, int ydt, int M, int N, int K, int G, int ng,
    int gshift, float* __restrict__ part, int slice_len, int ldy) {
    using Op = GsOp<T>;
    typedef typename Op::V V;
    constexpr int KC = KCS * 64;                 // k per LDS chunk
    constexpr int ROWB = KC * 2 + 16;            // LDS bytes per activation row (padded)
    constexpr int XROWS = TM * 16;
    constexpr int XPIECES = XROWS * KC / 8;      // 16-byte pieces per chunk
    constexpr int XPT = (XPIECES + 255) / 256;   // pieces per thread
    __shared__ __attribute__((aligned(16))) uint8_t sx[2][XROWS * ROWB];
    // TL: each wave's weight tiles regrouped, NW x [16 rows][256 bytes], 16-byte unit u of row r at u ^ r
    static_assert(!TL || KCS == 4, "transposed loads take a 256-code chunk");
    __shared__ __attribute__((aligned(16))) uint8_t wt[TL ? 4 * NW * 4096 : 16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // With a multiple of 8 blocks across N, block b covers row block (b & 7) * (nblk / 8) + (b >> 3):
    // blocks go round-robin over the 8 XCDs, so XCD x then writes one contiguous range of output
    // columns, which the split-K reduction reads back on the same XCD.
    const int nblk = gridDim.x;
    const int bx = (nblk & 7) == 0 ? (int)(blockIdx.x & 7) * (nblk >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
    const int nb = bx * (64 * NW) + wave * (16 * NW);   // this wave's first row
    const int kbeg = blockIdx.y * slice_len;
    const int kend = min(K, kbeg + slice_len);
    const int nchunks = (kend - kbeg + KC - 1) / KC;

    const __amdgpu_buffer_rsrc_t wrs = gs_rsrc(w, (uint32_t)N * (uint32_t)K);
    const uint32_t oob = (uint32_t)N * (uint32_t)K;
    const uint32_t kq = 16u * (uint32_t)(lane >> 4);            // lane's 16-code slot in a 64-k step
    // Per-tile row offsets of this lane (rows past N read out of range).
    uint32_t roff[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int n = nb + j * 16 + (lane & 15);
        roff[j] = n < N ? (uint32_t)n * (uint32_t)K : oob;
    }

    // ---- weight ring: one chunk (KCS steps x NW tiles) per buffer
    uint4 wa[KCS][NW], wb[KCS][NW];
    float sa[GMODE == GM_CHANNEL ? 1 : KCS][NW], sb[GMODE == GM_CHANNEL ? 1 : KCS][NW];
    auto issue = [&](uint4 (&buf)[KCS][NW], float (&sv)[GMODE == GM_CHANNEL ? 1 : KCS][NW], int chunk) {
        const int k0 = kbeg + chunk * KC;
#pragma unroll
        for (int st = 0; st < KCS; ++st) {
            const int ks = k0 + st * 64;
            const uint32_t kk = (uint32_t)ks + kq;
            const bool ok = chunk < nchunks && kk < (uint32_t)kend;
#pragma unroll
            for (int j = 0; j < NW; ++j) {
                if constexpr (TL) {
                    // load st of the chunk: rows 4 st .. 4 st + 3 of the tile, 256 contiguous bytes each
                    const int row = nb + j * 16 + 4 * st + (lane >> 4);
                    const uint32_t k2 = (uint32_t)k0 + 16u * (uint32_t)(lane & 15);
                    const bool ok2 = chunk < nchunks && k2 < (uint32_t)kend && row < N;
                    const uint32_t off = ok2 ? (uint32_t)row * (uint32_t)K + k2 : oob;
                    buf[st][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)off, 0, GS_NT));
                } else {
                    const uint32_t off = ok ? roff[j] + kk : oob;
                    buf[st][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)off, 0, GS_NT));
                }
                if constexpr (GMODE != GM_CHANNEL) {
                    const int n = min(nb + j * 16 + (lane & 15), N - 1);
                    const int g = ok ? (gshift >= 0 ? (int)(kk >> gshift) : (int)kk / G) : 0;
                    if constexpr (GMODE == GM_UE8M0) sv[st][j] = ue8m0_to_f32(((const uint8_t*)ws)[(size_t)n * ng + g]);
                    else sv[st][j] = ((const float*)ws)[(size_t)n * ng + g];
                }
            }
        }
    };

    // ---- activation chunk staging (registers -> LDS)
    uint4 xr[XPT];
    auto x_load = [&](int chunk) {
        const int k0 = kbeg + chunk * KC;
#pragma unroll
        for (int q = 0; q < XPT; ++q) {
            const int p = tid + q * 256;
            const int row = p / (KC / 8), col = (p % (KC / 8)) * 8;
            const int gk = k0 + col;
            xr[q] = (p < XPIECES && chunk < nchunks && row < M && gk < kend)
                        ? *(const uint4*)(x + (size_t)row * K + gk) : make_uint4(0, 0, 0, 0);
        }
    };
    auto x_store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < XPT; ++q) {
            const int p = tid + q * 256;
            if (p < XPIECES) {
                const int row = p / (KC / 8), col = (p % (KC / 8)) * 8;
                *(uint4*)&sx[buf][row * ROWB + col * 2] = xr[q];
            }
        }
    };

    f32x4 acc[TM][NW];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int j = 0; j < NW; ++j) acc[a][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint8_t* wtile = &wt[TL ? wave * NW * 4096 : 0];
    auto compute = [&](const uint4 (&buf)[KCS][NW], const float (&sv)[GMODE == GM_CHANNEL ? 1 : KCS][NW], int xb) {
        if constexpr (TL) {
            // The chunk's loads into this wave's tiles (LDS operations of one wave complete in order).
#pragma unroll
            for (int j = 0; j < NW; ++j)
#pragma unroll
                for (int st = 0; st < KCS; ++st) {
                    const int r = 4 * st + (lane >> 4);
                    *(uint4*)(wtile + j * 4096 + r * 256 + 16 * ((lane & 15) ^ r)) = buf[st][j];
                }
        }
#pragma unroll
        for (int st = 0; st < KCS; ++st) {
            V b1[NW], b2[NW];
#pragma unroll
            for (int j = 0; j < NW; ++j) {
                const float s = GMODE == GM_UE8M0 ? sv[st][j] : 1.f;
                // operand of step st: row lane & 15, 16-byte unit 4 st + (lane >> 4)
                const uint4 wv = TL ? *(const uint4*)(wtile + j * 4096 + (lane & 15) * 256 +
                                                      16 * ((4 * st + (lane >> 4)) ^ (lane & 15)))
                                    : buf[st][j];
                uint4 d1, d2;
                d1.x = Op::template cvt<FMT>(wv.x, s, false);
                d1.y = Op::template cvt<FMT>(wv.x, s, true);
                d1.z = Op::template cvt<FMT>(wv.y, s, false);
                d1.w = Op::template cvt<FMT>(wv.y, s, true);
                d2.x = Op::template cvt<FMT>(wv.z, s, false);
                d2.y = Op::template cvt<FMT>(wv.z, s, true);
                d2.z = Op::template cvt<FMT>(wv.w, s, false);
                d2.w = Op::template cvt<FMT>(wv.w, s, true);
                b1[j] = __builtin_bit_cast(V, d1);
                b2[j] = __builtin_bit_cast(V, d2);
            }
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const uint8_t* ap = &sx[xb][(a * 16 + (lane & 15)) * ROWB + (st * 64 + (int)kq) * 2];
                const V a1 = *(const V*)ap;
                const V a2 = *(const V*)(ap + 16);
#pragma unroll
                for (int j = 0; j < NW; ++j) {
                    if constexpr (GMODE == GM_F32) {
                        f32x4 t = Op::mma(a1, b1[j], f32x4{0.f, 0.f, 0.f, 0.f});
                        t = Op::mma(a2, b2[j], t);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[a][j][i] = fmaf(t[i], sv[st][j], acc[a][j][i]);
                    } else {
                        acc[a][j] = Op::mma(a1, b1[j], acc[a][j]);
                        acc[a][j] = Op::mma(a2, b2[j], acc[a][j]);
                    }
                }
            }
        }
    };

    // ---- pipeline. Issue order x(0) w(0) x(1) w(1) | x(2) w(2) | ...: the activation copy of a chunk
    // is issued before that chunk's weights, so writing it to LDS never waits for weights, and two
    // chunks of weights are in flight while one is consumed.
    x_load(0);
    issue(wa, sa, 0);
    x_store(0);
    x_load(1);
    issue(wb, sb, 1);
    __syncthreads();
    for (int c = 0; c < nchunks; c += 2) {
        compute(wa, sa, 0);
        x_store(1);
        if (c + 2 < nchunks) { x_load(c + 2); issue(wa, sa, c + 2); }
        __syncthreads();
        if (c + 1 >= nchunks) break;
        compute(wb, sb, 1);
        x_store(0);
        if (c + 3 < nchunks) { x_load(c + 3); issue(wb, sb, c + 3); }
        __syncthreads();
    }

    // ---- epilogue. MFMA 16x16 output: lane l holds rows 4(l>>4)+i, column l&15 of each tile.
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int n = nb + j * 16 + (lane & 15);
        if (n >= N) continue;
        if (part) {
            float* pp = part + (size_t)blockIdx.y * M * ldy;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = a * 16 + 4 * (lane >> 4) + i;
                    if (m < M) pp[(size_t)m * ldy + n] = acc[a][j][i];
                }
        } else {
            const float cs = GMODE == GM_CHANNEL ? (sk == TFP8_SCALE_UE8M0 ? ue8m0_to_f32(((const uint8_t*)ws)[n])
                                                                          : ((const float*)ws)[n])
                                                 : 1.f;
            const float bv = bias ? bias[n] : 0.f;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = a * 16 + 4 * (lane >> 4) + i;
                    if (m < M) {
                        const float v = acc[a][j][i] * cs;
                        store_elem(y, (size_t)m * ldy + n, ydt, xs ? fmaf(v, xs[m], bv) : v + bv);
                    }
                }
        }
    }
}

// ------------------------------------------------------------------ host side
namespace {

struct GsCfg { int tm, nw, kcs; };

// CU count of the current device, queried once per device (host threads may race to fill an
// entry with the same value, hence the atomic).
int gs_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cus[dev].load(std::memory_order_relaxed);
    if (!c) {
        int v = 0;
        c = (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v : 256;
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

}  // namespace

// Which scale handling a (G, scale kind) needs; -1 if this kernel does not take it.
int gemm_stream_gmode(int K, int G, int ws_kind) {
    if (G == K) return GM_CHANNEL;
    if (ws_kind == TFP8_SCALE_UE8M0) return GM_UE8M0;
    if (G % 64 == 0) return GM_F32;
    return -1;
}

// Tile config and split-K for an (M, N, K); the same function sizes the workspace.
// Above this many rows the LDS-tiled kernel (gemm.hip) reuses each weight tile better.
constexpr int GS_MAX_M = 128;

void gemm_stream_plan(int M, int N, int K, int G, int gmode, int* tm, int* nw, int* kcs, int* slices, int* slice_len) {
    // LDS per block = 2 * TM*16 * (KCS*128 + 16) bytes (gfx950 allows 160 KB per workgroup).
    // Configs by M from a sweep on MI355X (K = N = 8192); above 128 rows the LDS-tiled kernel wins.
    int T = (M + 15) / 16;
    int NWv = 1, KCSv = 4;
    if (T > 4) { NWv = 2; KCSv = 1; }
    else if (T > 2) { NWv = 2; KCSv = 2; }
    else if (T > 1) { NWv = 2; KCSv = 4; }
    T = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8;   // callers take this kernel only for M <= GS_MAX_M
    const int f_nw = tune(TUNE_GS_NW), f_kcs = tune(TUNE_GS_KCS);
    if (f_nw) NWv = f_nw;
    if (f_kcs) KCSv = f_kcs;
    const int KC = KCSv * 64;
    const int ntile = (N + 64 * NWv - 1) / (64 * NWv);
    // Split K until the grid covers the CUs ~2x, keeping slices whole chunks (and whole groups
    // for f32 group scales).
    int align = KC;
    if (gmode == GM_F32) { int a = KC, b = G; while (b) { int t = a % b; a = b; b = t; } align = KC / a * G; }
    int s = 1;
    const int want = 2 * gs_cus();
    while (ntile * s * 2 <= want && s < 8 && (K / (s * 2)) >= 2 * KC) s *= 2;
    const int fs = tune(TUNE_GS_SPLITK);
    if (fs > 0) s = std::min(fs, 8);
    int len = ((K + s - 1) / s + align - 1) / align * align;
    s = (K + len - 1) / len;
    *tm = T; *nw = NWv; *kcs = KCSv; *slices = s; *slice_len = len;
}

size_t gemm_stream_partial_bytes(int M, int N, int K, int G, int ws_kind) {
    const int gm = gemm_stream_gmode(K, G, ws_kind);
    if (gm < 0 || M > GS_MAX_M) return 0;
    int tm, nw, kcs, s, len;
    gemm_stream_plan(M, N, K, G, gm, &tm, &nw, &kcs, &s, &len);
    return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

template <typename T, int FMT, int TM, int NW, int KCS, int GMODE>
static void gs_launch(int slices, int slice_len, const void* x, const float* xs, const uint8_t* w, const void* ws,
                      int sk, const float* bias, void* y, int ydt, int M, int N, int K, int G, int ng, float* part,
                      hipStream_t s) {
    dim3 grid((N + 64 * NW - 1) / (64 * NW), slices);
    const int gshift = (G & (G - 1)) == 0 ? __builtin_ctz((unsigned)G) : -1;
    // 256-code chunks load as 4 rows x 256 contiguous bytes per instruction and are regrouped in LDS
    // (knob TFP8_GS_TL=0 keeps the 16 rows x 64 bytes operand layout).
    if constexpr (KCS == 4) {
        if (tune(TUNE_GS_TL)) {
            gemm_stream_kernel<T, FMT, TM, NW, KCS, GMODE, true><<<grid, 256, 0, s>>>(
                (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, part, slice_len, N);
            return;
        }
    }
    gemm_stream_kernel<T, FMT, TM, NW, KCS, GMODE, false><<<grid, 256, 0, s>>>((const T*)x, xs, w, ws, sk, bias, y, ydt,
                                                                              M, N, K, G, ng, gshift, part, slice_len, N);
}

template <typename T, int FMT, int GMODE>
static bool gs_dispatch(int tm, int nw, int kcs, int slices, int slice_len, const void* x, const float* xs,
                        const uint8_t* w, const void* ws, int sk, const float* bias, void* y, int ydt, int M, int N,
                        int K, int G, int ng, float* part, hipStream_t s) {
#define GS_CFG(TM_, NW_, KCS_)                                                                                  \
    if (tm == TM_ && nw == NW_ && kcs == KCS_) {                                                                \
        gs_launch<T, FMT, TM_, NW_, KCS_, GMODE>(slices, slice_len, x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, \
                                                 part, s);                                                      \
        return true;                                                                                            \
    }
    GS_CFG(1, 1, 4) GS_CFG(2, 2, 4) GS_CFG(4, 2, 2) GS_CFG(8, 2, 1)
    GS_CFG(1, 2, 4) GS_CFG(2, 1, 4) GS_CFG(4, 4, 2) GS_CFG(8, 4, 1)
#undef GS_CFG
    return false;
}

void splitk_reduce_launch(const float* part, int S, int M, int N, const void* ws, int sk, int colscale, const float* xs,
                          const float* bias, void* y, int ydt, int xcw, hipStream_t s);

// Runs the streaming GEMM if it takes this shape; returns NOT_TAKEN if it did not (caller falls back),
// 0 or an error code otherwise. x16 is f16/bf16 [M,K]; the matrix must be below 2^31 bytes.
int run_gemm_stream(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
                    const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype,
                    float* partial, hipStream_t s) {
    const int gm = gemm_stream_gmode(K, G, ws_kind);
    if (gm < 0 || M > GS_MAX_M || (long)N * K >= (1L << 31) || tune(TUNE_GEMM_V1)) return NOT_TAKEN;
    int tm, nw, kcs, slices, slice_len;
    gemm_stream_plan(M, N, K, G, gm, &tm, &nw, &kcs, &slices, &slice_len);
    float* part = slices > 1 ? partial : nullptr;
    const int ng = K / G;
    bool ok = false;
    if (x16_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, {
            if (gm == GM_CHANNEL) ok = gs_dispatch<__bf16, F, GM_CHANNEL>(tm, nw, kcs, slices, slice_len, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, part, s);
            else if (gm == GM_UE8M0) ok = gs_dispatch<__bf16, F, GM_UE8M0>(tm, nw, kcs, slices, slice_len, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, part, s);
            else ok = gs_dispatch<__bf16, F, GM_F32>(tm, nw, kcs, slices, slice_len, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, part, s);
        });
    } else {
        TFP8_DISPATCH_FMT(fmt, F, {
            if (gm == GM_CHANNEL) ok = gs_dispatch<_Float16, F, GM_CHANNEL>(tm, nw, kcs, slices, slice_len, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, part, s);
            else if (gm == GM_UE8M0) ok = gs_dispatch<_Float16, F, GM_UE8M0>(tm, nw, kcs, slices, slice_len, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, part, s);
            else ok = gs_dispatch<_Float16, F, GM_F32>(tm, nw, kcs, slices, slice_len, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G, ng, part, s);
        });
    }
    if (!ok) return NOT_TAKEN;
    int rc = check_launch("tfp8_gemm (stream)");
    if (rc || slices <= 1) return rc;
    const int nblk = (N + 64 * nw - 1) / (64 * nw);
    const int xcw = nblk % 8 == 0 ? nblk / 8 * 64 * nw : 0;
    splitk_reduce_launch(part, slices, M, N, ws, ws_kind, gm == GM_CHANNEL ? 1 : 0, xs, bias, y, y_dtype, xcw, s);
    return check_launch("tfp8_gemm (stream) splitk reduce");
}

}  // namespace tfp8
