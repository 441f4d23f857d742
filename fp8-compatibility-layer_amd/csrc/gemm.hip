// LDS-tiled FP8-weight GEMM on gfx950 MFMA (M > 8 rows).
//
// y[m,n] = xs[m] * sum_g s(n,g) * sum_{k in g} x[m,k] * decode(w[n,k]) + bias[n]
// (reference gemm_w8a16, tfp8/csrc/tfp8_kernels.cu:271-411), built for CDNA4:
//   * block tile BM x BN x 64, 4 waves in a WM x WN grid, wave tile (BM/WM) x (BN/WN) made of
//     16x16 outputs of v_mfma_f32_16x16x32_{f16,bf16} (fp32 accumulation);
//   * per 64-wide K step the activation tile (f16/bf16) and the raw FP8 weight tile (1 byte per
//     element, half the LDS footprint of a decoded tile) are staged through registers into a
//     double-buffered LDS pair; each wave reads its 8-byte B fragments from LDS and decodes
//     them in registers with v_cvt_scalef32_pk_{f16,bf16}_{fp8,bf8} right before the MFMA, so
//     the weight is never written back decoded, to LDS or to HBM;
//   * per-channel scales (one group) are applied in the epilogue; K-group scales (G % 32 == 0)
//     multiply an fp32 partial accumulator at every group boundary (exact for any f32 scale,
//     no folding of scales into 16-bit weights);
//   * tiles are walked so that blocks sharing a weight column tile are dispatched to the same
//     XCD (blocks go round-robin over the 8 XCDs, each with its own L2);
//   * optional split-K over gridDim.y writes fp32 partial sums into the caller's workspace and a
//     second kernel reduces them and applies the epilogue.
#include <algorithm>

#include "tfp8_common.h"

namespace tfp8 {

constexpr int GEMM_BK = 64;
constexpr int A_ROW_BYTES = GEMM_BK * 2 + 16;   // 144: 16-byte pad keeps ds_read_b128 conflict-free
constexpr int B_ROW_BYTES = GEMM_BK + 16;       // 80

template <typename T> struct MfmaOp;
template <> struct MfmaOp<_Float16> {
    typedef f16x8 V;
    static __device__ __forceinline__ f32x4 run(V a, V b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, bool hi) { return cvt2_f16<FMT>(w, hi); }
};
template <> struct MfmaOp<__bf16> {
    typedef bf16x8 V;
    static __device__ __forceinline__ f32x4 run(V a, V b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, bool hi) { return cvt2_bf16<FMT>(w, hi); }
};

// 8 FP8 codes (k order) -> one MFMA B operand (8 x 16-bit).
template <typename T, int FMT>
__device__ __forceinline__ typename MfmaOp<T>::V decode_frag(uint2 raw) {
    uint4 u;
    u.x = MfmaOp<T>::template cvt<FMT>(raw.x, false);
    u.y = MfmaOp<T>::template cvt<FMT>(raw.x, true);
    u.z = MfmaOp<T>::template cvt<FMT>(raw.y, false);
    u.w = MfmaOp<T>::template cvt<FMT>(raw.y, true);
    return __builtin_bit_cast(typename MfmaOp<T>::V, u);
}

__device__ __forceinline__ float scale_at(const void* ws, int sk, size_t i) {
    return sk == TFP8_SCALE_UE8M0 ? ue8m0_to_f32(((const uint8_t*)ws)[i]) : ((const float*)ws)[i];
}

template <typename T, int FMT, int BM, int BN, int WM, int WN, bool GROUPED>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(
    const T* __restrict__ x, const float* __restrict__ xs, const uint8_t* __restrict__ w,
    const void* __restrict__ ws, int sk, const float* __restrict__ bias, void* __restrict__ y, int ydt,
    int M, int N, int K, int G, int ng, float* __restrict__ part, int slice_len) {
    using Op = MfmaOp<T>;
    typedef typename Op::V V;
    constexpr int NT = 64 * WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 16, TN = WTN / 16;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 16x16 MFMA tile");
    constexpr int A_CHUNKS = BM * (GEMM_BK / 8);    // 16-byte chunks of the activation tile
    constexpr int B_CHUNKS = BN * (GEMM_BK / 16);   // 16-byte chunks of the FP8 weight tile
    constexpr int CA = (A_CHUNKS + NT - 1) / NT;
    constexpr int CB = (B_CHUNKS + NT - 1) / NT;

    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * A_ROW_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * B_ROW_BYTES];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // XCD-aware tile order: consecutive ids land on one XCD, and consecutive ids walk M first,
    // so blocks that read the same weight tile share an L2.
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN, nt = ntm * ntn;
    int id = blockIdx.x;
    if ((nt & 7) == 0) id = (blockIdx.x & 7) * (nt >> 3) + (blockIdx.x >> 3);
    const int m0 = (id % ntm) * BM, n0 = (id / ntm) * BN;

    const int kbeg = blockIdx.y * slice_len;
    const int kend = min(K, kbeg + slice_len);

    uint4 ra[CA], rb[CB];
    auto load_tile = [&](int kt) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * NT;
            const int row = c >> 3, col = (c & 7) * 8;
            const int gm = m0 + row, gk = kt + col;
            ra[i] = (c < A_CHUNKS && gm < M && gk < kend) ? *(const uint4*)(x + (size_t)gm * K + gk)
                                                          : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = tid + i * NT;
            const int row = c >> 2, col = (c & 3) * 16;
            const int gn = n0 + row, gk = kt + col;
            rb[i] = (c < B_CHUNKS && gn < N && gk < kend) ? *(const uint4*)(w + (size_t)gn * K + gk)
                                                          : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * NT;
            if (c < A_CHUNKS) *(uint4*)&sA[buf][(c >> 3) * A_ROW_BYTES + (c & 7) * 16] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = tid + i * NT;
            if (c < B_CHUNKS) *(uint4*)&sB[buf][(c >> 2) * B_ROW_BYTES + (c & 3) * 16] = rb[i];
        }
    };

    f32x4 acc[TM][TN];
    f32x4 prt[GROUPED ? TM : 1][GROUPED ? TN : 1];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (GROUPED) {
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) prt[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Columns this lane accumulates (one per TN sub-tile), clamped for scale loads.
    int colc[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b) colc[b] = min(n0 + wn * WTN + b * 16 + (lane & 15), N - 1);

    int gidx = 0, gnext = 0;
    float gs[GROUPED ? TN : 1];
    if constexpr (GROUPED) {
        gidx = kbeg / G;
        gnext = (gidx + 1) * G;
#pragma unroll
        for (int b = 0; b < TN; ++b) gs[b] = scale_at(ws, sk, (size_t)colc[b] * ng + gidx);
    }

    const int arow = wm * WTM + (lane & 15);
    const int brow = wn * WTN + (lane & 15);
    const int kq = 8 * (lane >> 4);   // this lane's 8-wide K slot inside a 32-wide MFMA step

    load_tile(kbeg);
    store_tile(0);
    __syncthreads();

    int buf = 0;
    for (int kt = kbeg; kt < kend; kt += GEMM_BK) {
        const bool more = kt + GEMM_BK < kend;
        if (more) load_tile(kt + GEMM_BK);
#pragma unroll
        for (int ks = 0; ks < GEMM_BK / 32; ++ks) {
            const int kk = kt + ks * 32;
            if (kk < kend) {
                V af[TM], bf[TN];
#pragma unroll
                for (int a = 0; a < TM; ++a)
                    af[a] = *(const V*)&sA[buf][(arow + a * 16) * A_ROW_BYTES + (ks * 32 + kq) * 2];
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    bf[b] = decode_frag<T, FMT>(*(const uint2*)&sB[buf][(brow + b * 16) * B_ROW_BYTES + ks * 32 + kq]);
#pragma unroll
                for (int a = 0; a < TM; ++a)
#pragma unroll
                    for (int b = 0; b < TN; ++b) {
                        if constexpr (GROUPED) prt[a][b] = Op::run(af[a], bf[b], prt[a][b]);
                        else acc[a][b] = Op::run(af[a], bf[b], acc[a][b]);
                    }
                if constexpr (GROUPED) {
                    if (kk + 32 == gnext || kk + 32 >= kend) {
#pragma unroll
                        for (int a = 0; a < TM; ++a)
#pragma unroll
                            for (int b = 0; b < TN; ++b) {
#pragma unroll
                                for (int i = 0; i < 4; ++i) acc[a][b][i] = fmaf(prt[a][b][i], gs[b], acc[a][b][i]);
                                prt[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
                            }
                        gidx = min(gidx + 1, ng - 1);
                        gnext += G;
#pragma unroll
                        for (int b = 0; b < TN; ++b) gs[b] = scale_at(ws, sk, (size_t)colc[b] * ng + gidx);
                    }
                }
            }
        }
        if (more) store_tile(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // Epilogue.  MFMA 16x16 output layout: lane l holds rows 4*(l>>4)+i, column l&15.
    const int rbase = m0 + wm * WTM + 4 * (lane >> 4);
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int col = n0 + wn * WTN + b * 16 + (lane & 15);
        if (col >= N) continue;
        if (part) {
            float* pp = part + (size_t)blockIdx.y * M * N;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = rbase + a * 16 + i;
                    if (row < M) pp[(size_t)row * N + col] = acc[a][b][i];
                }
        } else {
            const float cs = GROUPED ? 1.f : scale_at(ws, sk, (size_t)col);
            const float bv = bias ? bias[col] : 0.f;
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = rbase + a * 16 + i;
                    if (row < M) {
                        const float v = acc[a][b][i] * cs;
                        store_elem(y, (size_t)row * N + col, ydt, xs ? fmaf(v, xs[row], bv) : v + bv);
                    }
                }
        }
    }
}

// Split-K epilogue: y = (sum_s part[s]) * colscale * xs + bias.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                                            const void* __restrict__ ws, int sk, int colscale,
                                                            const float* __restrict__ xs,
                                                            const float* __restrict__ bias, void* __restrict__ y,
                                                            int ydt) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        float v = 0.f;
        for (int s = 0; s < S; ++s) v += part[(size_t)s * total + i];
        const int row = (int)(i / N), col = (int)(i % N);
        if (colscale) v *= scale_at(ws, sk, (size_t)col);
        const float bv = bias ? bias[col] : 0.f;
        store_elem(y, (size_t)i, ydt, xs ? fmaf(v, xs[row], bv) : v + bv);
    }
}

// ------------------------------------------------------------------ planning
struct GemmPlan {
    int bm, bn, wm, wn;   // tile config
    int slices;           // split-K factor (1 = none)
};

static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Tile config by M; split K when the tile grid would leave CUs idle and the fp32 partials stay
// small next to the weight stream.
GemmPlan gemm_plan(int M, int N, int K) {
    GemmPlan p;
    if (M <= 16) p = {16, 64, 1, 4, 1};
    else if (M <= 32) p = {32, 64, 2, 2, 1};
    else if (M <= 64) p = {64, 64, 2, 2, 1};
    else if (M <= 128) p = {64, 128, 2, 2, 1};
    else p = {128, 128, 2, 2, 1};
    const int forced = env_int("TFP8_GEMM_TILE", 0);   // tuning hook: 1..5 picks a config above
    if (forced == 1) p = {16, 64, 1, 4, 1};
    else if (forced == 2) p = {32, 64, 2, 2, 1};
    else if (forced == 3) p = {64, 64, 2, 2, 1};
    else if (forced == 4) p = {64, 128, 2, 2, 1};
    else if (forced == 5) p = {128, 128, 2, 2, 1};
    const long tiles = (long)((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
    int s = 1;
    // Split K until the grid covers the CUs (measured best: 4 slices for 8192^2 at M=256).
    while (tiles * s < 256 && s < 8 && (K / (s * 2)) >= 512) s *= 2;
    const int fs = env_int("TFP8_GEMM_SPLITK", 0);
    if (fs > 0) s = fs;
    p.slices = s;
    return p;
}

size_t gemm_stream_partial_bytes(int M, int N, int K, int G, int ws_kind);

// Workspace for either GEMM kernel's split-K partials (the streaming kernel's split is sized
// with per-channel alignment, an upper bound for every group size).
size_t gemm_partial_bytes(int M, int N, int K) {
    const GemmPlan p = gemm_plan(M, N, K);
    const size_t v1 = p.slices > 1 ? (size_t)p.slices * M * N * sizeof(float) : 0;
    return std::max(v1, gemm_stream_partial_bytes(M, N, K, K, TFP8_SCALE_F32));
}

void splitk_reduce_launch(const float* part, int S, int M, int N, const void* ws, int sk, int colscale, const float* xs,
                          const float* bias, void* y, int ydt, hipStream_t s) {
    const unsigned grid = grid_for((int64_t)M * N, 256);
    splitk_reduce_kernel<<<grid, 256, 0, s>>>(part, S, M, N, ws, sk, colscale, xs, bias, y, ydt);
}

int run_gemm_stream(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
                    const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype,
                    float* partial, hipStream_t s);

template <typename T, int FMT, int BM, int BN, int WM, int WN>
static void launch_gemm_cfg(const void* x, const float* xs, const uint8_t* w, const void* ws, int sk,
                            const float* bias, void* y, int ydt, int M, int N, int K, int G, int ng, float* part,
                            int slices, int slice_len, hipStream_t s) {
    const int nt = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    dim3 grid(nt, slices);
    if (ng > 1)
        gemm_kernel<T, FMT, BM, BN, WM, WN, true><<<grid, 64 * WM * WN, 0, s>>>(
            (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, part, slice_len);
    else
        gemm_kernel<T, FMT, BM, BN, WM, WN, false><<<grid, 64 * WM * WN, 0, s>>>(
            (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, part, slice_len);
}

template <typename T, int FMT>
static void launch_gemm_t(const GemmPlan& p, const void* x, const float* xs, const uint8_t* w, const void* ws,
                          int sk, const float* bias, void* y, int ydt, int M, int N, int K, int G, int ng,
                          float* part, int slices, int slice_len, hipStream_t s) {
#define TFP8_GEMM_CFG(BM_, BN_, WM_, WN_)                                                                    \
    if (p.bm == BM_ && p.bn == BN_ && p.wm == WM_ && p.wn == WN_) {                                         \
        launch_gemm_cfg<T, FMT, BM_, BN_, WM_, WN_>(x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, part,     \
                                                    slices, slice_len, s);                                  \
        return;                                                                                             \
    }
    TFP8_GEMM_CFG(16, 64, 1, 4)
    TFP8_GEMM_CFG(32, 64, 2, 2)
    TFP8_GEMM_CFG(64, 64, 2, 2)
    TFP8_GEMM_CFG(64, 128, 2, 2)
    TFP8_GEMM_CFG(128, 128, 2, 2)
#undef TFP8_GEMM_CFG
}

static int gcd_i(int a, int b) { while (b) { int t = a % b; a = b; b = t; } return a; }

// Validated by the caller.  x16 is f16 or bf16 [M,K]; xs optional.  partial: workspace of
// gemm_partial_bytes() (may be null when that is 0).
int run_gemm(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
             const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, float* partial,
             hipStream_t s) {
    // The weight-streaming kernel takes most shapes; the LDS-tiled kernel below is the general path.
    const int rs = run_gemm_stream(x16, x16_dtype, xs, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, partial, s);
    if (rs != 1) return rs;
    const int ng = K / G;
    GemmPlan p = gemm_plan(M, N, K);
    int slices = p.slices, slice_len = K;
    if (slices > 1) {
        // Slices are whole 64-wide K tiles, and whole K groups when the scales are grouped.
        int align = GEMM_BK;
        if (ng > 1) align = GEMM_BK / gcd_i(GEMM_BK, G) * G;
        slice_len = ((K + slices - 1) / slices + align - 1) / align * align;
        slices = (K + slice_len - 1) / slice_len;
        if (slices <= 1) { slices = 1; slice_len = K; }
    }
    float* part = slices > 1 ? partial : nullptr;
    if (x16_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, launch_gemm_t<__bf16, F>(p, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K, G,
                                                          ng, part, slices, slice_len, s));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, launch_gemm_t<_Float16, F>(p, x16, xs, w, ws, ws_kind, bias, y, y_dtype, M, N, K,
                                                            G, ng, part, slices, slice_len, s));
    }
    int rc = check_launch("tfp8_gemm");
    if (rc || slices <= 1) return rc;
    const unsigned grid = grid_for((int64_t)M * N, 256);
    splitk_reduce_kernel<<<grid, 256, 0, s>>>(part, slices, M, N, ws, ws_kind, ng == 1 ? 1 : 0, xs, bias, y,
                                              y_dtype);
    return check_launch("tfp8_gemm splitk reduce");
}

}  // namespace tfp8
