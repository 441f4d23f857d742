// W8A8: FP8 activations x FP8 weights with 32-wide K-block scales (reference fp8_cuda.py and
// fp8_gemm_kernel.cu), on gfx950 matrix cores.
//
//   quantize:  per row and 32-wide K block, s = max(amax / max_finite, 1e-12); with UE8M0,
//              e = clamp(ceil(log2 s), -127, 127), s = 2^e and the stored byte is e + 127;
//              q = encode(clamp(x / s, +-max_finite))                      (fp8_cuda.py:74-92)
//   GEMM:      C[m,n] = sum_kb sa[m,kb] * sb[n,kb] * sum_{k in kb} A[m,k] * B[k,n] + bias[n]
//              (block mode), or (sum_k A B) * sa[m] * sb[n] + bias[n] (row/col mode)
//                                                                      (fp8_gemm_kernel.cu:41-118)
//
// The weight operand is taken transposed, Bt[N,K] (k contiguous, as the quantizer writes it):
// both matrix-core operands then load as contiguous k runs.  The GEMM kernels and their numerics
// are described at the GEMM section below.
#include <type_traits>

#include "tfp8_common.h"

namespace tfp8 {

namespace {

constexpr uint32_t W8_FLAGS = 0x00020000u;
constexpr uint32_t W8_OOB = 0x80000000u;
enum { W8_BLOCK = 0, W8_ROWCOL = 1 };

template <int FA, int FB>
__device__ __forceinline__ f32x4 w8_mma(long a, long b, f32x4 c) {
    if constexpr (FA == TFP8_E4M3FN && FB == TFP8_E4M3FN) return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
    else if constexpr (FA == TFP8_E4M3FN) return __builtin_amdgcn_mfma_f32_16x16x32_fp8_bf8(a, b, c, 0, 0, 0);
    else if constexpr (FB == TFP8_E4M3FN) return __builtin_amdgcn_mfma_f32_16x16x32_bf8_fp8(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_bf8_bf8(a, b, c, 0, 0, 0);
}

template <bool UE8M0>
__device__ __forceinline__ float w8_scale(const void* p, size_t i) {
    if constexpr (UE8M0) return ue8m0_to_f32(((const uint8_t*)p)[i]);
    else return ((const float*)p)[i];
}

// ------------------------------------------------------------------ quantizer
// One thread per 32-value block (the blocks of a row are consecutive in memory).  A block holding
// a NaN gets a NaN scale (UE8M0 byte 255, the kernel contract's NaN) and NaN codes 0x7F, as
// torch's amax and division propagate it; an infinite amax gives scale inf (UE8M0: 2^127).
template <int FMT, int XDT, bool UE8M0>
__global__ __launch_bounds__(256) void w8_quantize_kernel(const void* __restrict__ x, int R, int K,
                                                          uint8_t* __restrict__ q, void* __restrict__ scale) {
    using F = Fmt<FMT>;
    const int kb_n = K / 32;
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (int64_t)R * kb_n) return;
    const size_t base = (size_t)blk * 32;   // row-major [R, K]: block blk starts at element 32*blk
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = load_elem<XDT>(x, base + i);
    float amax = 0.f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        amax = fmaxf(amax, fabsf(v[i]));     // fmaxf skips NaN operands: they are tracked apart
        nan |= v[i] != v[i];
    }
    float s = nan ? __builtin_nanf("") : fmaxf(amax / F::MAX_FINITE, 1e-12f);
    if constexpr (UE8M0) {
        uint8_t byte = 0xFFu;
        if (!nan) {
            int e = 127;
            if (s != __builtin_inff()) {
                int ex;
                const float m = frexpf(s, &ex);  // s = m * 2^ex, m in [0.5, 1): ceil(log2 s) exactly
                e = max(-127, min(127, m == 0.5f ? ex - 1 : ex));
            }
            s = ldexpf(1.f, e);
            byte = (uint8_t)(e + 127);
        }
        ((uint8_t*)scale)[blk] = byte;
    } else {
        ((float*)scale)[blk] = s;
    }
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float d = v[4 * i + j] / s;
            const uint32_t code = d != d ? 0x7Fu : encode_fp8<FMT>(fminf(fmaxf(d, -F::MAX_FINITE), F::MAX_FINITE));
            word |= code << (8 * j);
        }
        w[i] = word;
    }
    uint4* dst = (uint4*)(q + base);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// ------------------------------------------------------------------ GEMM
// Three kernels share the tiling below and differ in what the matrix cores multiply:
//
//   w8_bf16_kernel (default for UE8M0 block scales and row/column scales): FP8 codes are decoded
//     to bf16 once per tile with the UE8M0 block scale folded into the decode (exact), and
//     v_mfma_f32_16x16x32_bf16 accumulates exact products in fp32.
//   w8_f16_kernel (default for FP32 block scales): FP8 codes are decoded to f16 once per tile
//     (exact: every FP8 value is an f16) and multiplied by v_mfma_f32_16x16x32_f16, whose products
//     reach the fp32 accumulator exactly -- the numerics of the reference's fp16 WMMA
//     (fp8_gemm_kernel.cu:72-99).  One MFMA covers exactly one 32-wide scale block of a 16 x 16
//     tile; its result is multiplied by sa * sb and accumulated in fp32 (fp8_gemm_kernel.cu:74-93).
//   w8_mx_kernel (native FP8): the codes go to the FP8 matrix cores as they are.  Those align
//     the products of one dot product to the largest and keep about 13 fraction bits (measured:
//     2^16 + 2^0 sums to 2^16), so results differ from an fp32 sum by ~1e-5..1e-4 of max|C|.
//     UE8M0 block scales ride in v_mfma_scale_f32_16x16x128_f8f6f4 (one E8M0 byte per lane);
//     row/column scales use the unscaled instruction; FP32 block scales use four
//     v_mfma_f32_16x16x32 per 128-step with the fp32 multiply-accumulate above.
//
// Tiling: block tile BT x BT of C split over a grid of waves, each owning TI x TJ MFMA tiles of
// 16 x 16; K advances 64 per step (128 in the native kernel).  Each step's A and Bt tiles (BT rows
// x the step's codes, k contiguous) are loaded into registers one step ahead and written (decoded,
// for the f16 and bf16 kernels) to the other half of a double-buffered LDS pair, so one barrier
// per step suffices.
// Out-of-range rows and the K tail read as zero through buffer-load bounds.
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// XCD-aware tile order: consecutive blocks go to the 8 XCDs in turn; renumber so each XCD owns a
// contiguous run, then walk that run in groups of 8 tile rows so co-resident blocks share A and
// Bt panels in their XCD's L2.
__device__ __forceinline__ void w8_tile(int M, int N, int BT, int& m0, int& n0) {
    const int nbm = (M + BT - 1) / BT, nbn = (N + BT - 1) / BT, nblk = nbm * nbn;
    const int xcd = blockIdx.x & 7, q8 = nblk >> 3, r8 = nblk & 7;
    const int lb = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    constexpr int GM = 8;
    const int grp = lb / (GM * nbn), first = grp * GM, gsz = min(nbm - first, GM), in = lb % (GM * nbn);
    m0 = (first + in % gsz) * BT;
    n0 = (in / gsz) * BT;
}

// Per-step operand loader: BT rows x 128 codes of A (op 0) and Bt (op 1), CH 16-byte chunks per
// thread and operand, plus (block mode) the step's 4 scales per row as fp32 words.
template <int BT, bool UE8M0, bool BLOCK_SCALES, int NT = 256>
struct W8Loader {
    static constexpr int CH = BT * 8 / NT;
    static constexpr int NSW = BLOCK_SCALES ? 2 * BT * 4 / NT : 1;
    static_assert(BT * 8 % NT == 0 && (!BLOCK_SCALES || BT * 4 % NT == 0),
                  "tile chunks and scale words of one operand must fill whole thread sweeps");
    __amdgpu_buffer_rsrc_t rs[2], rss[2];
    int K, nkb;
    uint4 rt[2][CH];
    float rsc[NSW];

    __device__ __forceinline__ W8Loader(const uint8_t* a, const void* sa, const uint8_t* bt, const void* sb, int M,
                                        int N, int K_, int m0, int n0)
        : K(K_), nkb(K_ / 32) {
        const uint32_t ra = (uint32_t)min(BT, M - m0), rb = (uint32_t)min(BT, N - n0);
        rs[0] = __builtin_amdgcn_make_buffer_rsrc((void*)(a + (size_t)m0 * K), (short)0, (int)(ra * (uint32_t)K),
                                                  (int)W8_FLAGS);
        rs[1] = __builtin_amdgcn_make_buffer_rsrc((void*)(bt + (size_t)n0 * K), (short)0, (int)(rb * (uint32_t)K),
                                                  (int)W8_FLAGS);
        constexpr int SB = UE8M0 ? 1 : 4;
        rss[0] = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)sa + (size_t)m0 * nkb * SB), (short)0,
                                                   (int)(ra * (uint32_t)nkb * SB), (int)W8_FLAGS);
        rss[1] = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)sb + (size_t)n0 * nkb * SB), (short)0,
                                                   (int)(rb * (uint32_t)nkb * SB), (int)W8_FLAGS);
    }
    __device__ __forceinline__ void load(int kt, int tid) {
#pragma unroll
        for (int op = 0; op < 2; ++op)
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int ch = tid + i * NT, row = ch >> 3, col = (ch & 7) * 16;
                const uint32_t off = kt + col < K ? (uint32_t)row * (uint32_t)K + (uint32_t)(kt + col) : W8_OOB;
                rt[op][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs[op], (int)off, 0, 0));
            }
        if constexpr (BLOCK_SCALES) {
            const int kb0 = kt / 32;
#pragma unroll
            for (int i = 0; i < NSW; ++i) {
                // BT * 4 is a multiple of NT and tid < NT: the operand depends on i only
                const int w = tid + i * NT, op = i * NT / (BT * 4), row = (w >> 2) % BT, q = w & 3;
                const bool ok = kb0 + q < nkb;
                if constexpr (UE8M0) {
                    const uint32_t o = ok ? (uint32_t)(row * nkb + kb0 + q) : W8_OOB;
                    rsc[i] = ue8m0_to_f32((uint8_t)__builtin_amdgcn_raw_buffer_load_b8(rss[op], (int)o, 0, 0));
                } else {
                    const uint32_t o = ok ? (uint32_t)((row * nkb + kb0 + q) * 4) : W8_OOB;
                    rsc[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rss[op], (int)o, 0, 0));
                }
            }
        }
    }
};

// Epilogue: C[m, n] = acc (+ row/column scales) + bias[n], fp32, row-major.  The wave owns rows
// wm * WTM + i * 16 + 4 (lane >> 4) + r and columns wn * WTN + j * 16 + (lane & 15).
template <int TI, int TJ, int WTM, int WTN, bool UE8M0, int MODE>
__device__ __forceinline__ void w8_store(f32x4 (&acc)[TI][TJ], const void* sa, const void* sb, const float* bias,
                                         float* c, int M, int N, int m0, int n0, int wm, int wn, int lane) {
    const int frow = lane & 15, orow = 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int n = n0 + wn * WTN + j * 16 + frow;
        if (n >= N) continue;
        const float bv = bias ? bias[n] : 0.f;
        const float cs = MODE == W8_ROWCOL ? w8_scale<UE8M0>(sb, (size_t)n) : 1.f;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * WTM + i * 16 + orow + r;
                if (m >= M) continue;
                float v = acc[i][j][r];
                if constexpr (MODE == W8_ROWCOL) v = v * w8_scale<UE8M0>(sa, (size_t)m) * cs;
                c[(size_t)m * N + n] = v + bv;
            }
    }
}

// ---- exact kernel for FP32 block scales: f16 tiles in LDS.  128 x 128 tile, 8 waves of 64 x 32,
// K steps of 64.  The codes are decoded to f16 once per block on their way into a double-buffered
// LDS pair (2 x 2 x 16 KB); a row of a tile is 64 halves = 8 chunks of 8, chunk u of row r at
// u ^ ((r >> 1) & 7), so the 16 rows one fragment read touches land on distinct bank groups.
// Lane l of an MFMA for scale block q reads row l & 15, chunk 4q + (l >> 4): k = 32q + 8 (l >> 4)
// + 0..7, the instruction's own k order.  Each MFMA result (one 32-block of a 16 x 16 tile) is
// multiplied by sa * sb and added to the fp32 accumulator (fp8_gemm_kernel.cu:74-93: the product
// sa * sb rounded to fp32, then one fused multiply-add, as racc += partial * s).
//
// The scale arithmetic (two VALU ops per output element and 32-block) is what bounds this kernel,
// so the step is built to keep the VALU fed and the register count at 124 (two blocks per CU, four
// waves per SIMD):
//   * the A scales of a step take one 8-byte LDS read per lane: lane (g, k) (g = lane >> 4,
//     k = lane & 15) holds the (q = 0, 1) pair of row 16 (k >> 2) + 4 g + (k & 3) of the wave tile,
//     and the multiply for row tile i, value r of any lane in lane row g takes it from lane
//     k = 4 i + r of its row of 16 with DPP row_newbcast inside the v_mul_f32 itself;
//   * the MFMAs of row tile i + 1 are issued between the multiply-adds of row tile i (pinned with
//     scheduling barriers), and row tile i + 2's fragments are read from LDS during row tile i;
//   * the K loop is unrolled by two, so each step's LDS buffer is a constant and every LDS address
//     a loop-invariant register plus an immediate; global loads take loop-invariant lane offsets
//     with the K position in soffset, bounds-checked only for a partial last tile.
// 8192^3 on one box: 2650 us for the previous form of this kernel (four A-scale LDS reads per
// row tile, MFMA results consumed right after each MFMA, 154 VGPRs: one block per CU) against
// 1915-1945 us, bit-identical outputs over the parity shapes.

// sa(lane n of this lane's row of 16) * sb as one v_mul_f32_dpp with row_newbcast:n; n is a
// constant after unrolling.  sa comes straight from an LDS read (no VALU write feeds the DPP read).
__device__ __forceinline__ float w8_mul_bcast(float sa, float sb, int n) {
    float r;
    switch (n) {
#define W8_RB(k) case k: asm("v_mul_f32_dpp %0, %1, %2 row_newbcast:" #k " row_mask:0xf bank_mask:0xf bound_ctrl:1" \
                             : "=v"(r) : "v"(sa), "v"(sb)); break;
        W8_RB(0) W8_RB(1) W8_RB(2) W8_RB(3) W8_RB(4) W8_RB(5) W8_RB(6) W8_RB(7)
        W8_RB(8) W8_RB(9) W8_RB(10) W8_RB(11) W8_RB(12) W8_RB(13) W8_RB(14) default: W8_RB(15)
#undef W8_RB
    }
    return r;
}

template <int FA, int FB>
__global__ __launch_bounds__(512) void w8_f16_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ sa, const uint8_t* __restrict__ bt,
    const float* __restrict__ sb, const float* __restrict__ bias, float* __restrict__ c, int M, int N, int K) {
    constexpr int BT = 128, WM = 2, WN = 4, WTM = BT / WM, WTN = BT / WN, TI = WTM / 16, TJ = WTN / 16;
    constexpr int NT = 64 * WM * WN, KS = 64, CH = BT * (KS / 16) / NT;
    static_assert(CH == 1 && 2 * BT * 2 == NT && TI == 4, "one chunk per thread and operand, one scale word per thread");
    __shared__ __attribute__((aligned(16))) uint8_t sT[2][2][BT * 128];   // [buffer][A, Bt][row * 128 B]
    __shared__ __attribute__((aligned(16))) float sS[2][2][BT * 2];       // [buffer][A, Bt][row * 2 + q]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int m0, n0;
    w8_tile(M, N, BT, m0, n0);
    const int nkb = K / 32, ntile = (K + KS - 1) / KS;
    const uint32_t rows[2] = {(uint32_t)min(BT, M - m0), (uint32_t)min(BT, N - n0)};
    __amdgpu_buffer_rsrc_t rs[2], rss[2];
    rs[0] = __builtin_amdgcn_make_buffer_rsrc((void*)(a + (size_t)m0 * K), (short)0, (int)(rows[0] * (uint32_t)K),
                                              (int)W8_FLAGS);
    rs[1] = __builtin_amdgcn_make_buffer_rsrc((void*)(bt + (size_t)n0 * K), (short)0, (int)(rows[1] * (uint32_t)K),
                                              (int)W8_FLAGS);
    rss[0] = __builtin_amdgcn_make_buffer_rsrc((void*)(sa + (size_t)m0 * nkb), (short)0,
                                               (int)(rows[0] * (uint32_t)nkb * 4u), (int)W8_FLAGS);
    rss[1] = __builtin_amdgcn_make_buffer_rsrc((void*)(sb + (size_t)n0 * nkb), (short)0,
                                               (int)(rows[1] * (uint32_t)nkb * 4u), (int)W8_FLAGS);

    // Thread tid loads codes k = kt + 16 (tid & 3) .. +15 of row tid >> 2 of both operands, and one
    // scale word: threads 0..255 A's, 256..511 Bt's (the operand is wave-uniform), word w = tid & 255
    // = row w >> 1, block kt / 32 + (w & 1).  Past K and past the block's rows the loads read zeros.
    const int s_op = wave >> 2, s_w = tid & 255;
    const int ld_row = tid >> 2, ld_k = 16 * (tid & 3);
    const uint32_t ld_off = (uint32_t)ld_row * (uint32_t)K + (uint32_t)ld_k;
    const uint32_t sc_off = (uint32_t)(((s_w >> 1) * nkb + (s_w & 1)) * 4);
    uint4 rt[2];
    float rsc;
    auto load = [&](int kt) {
        if (kt + KS <= K) {   // a whole tile: no per-lane bounds
#pragma unroll
            for (int op = 0; op < 2; ++op)
                rt[op] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs[op], (int)ld_off, kt, 0));
            rsc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rss[s_op], (int)sc_off, (kt / 32) * 4, 0));
        } else {
            const uint32_t off = kt + ld_k < K ? ld_off + (uint32_t)kt : W8_OOB;
#pragma unroll
            for (int op = 0; op < 2; ++op)
                rt[op] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs[op], (int)off, 0, 0));
            const uint32_t o = kt / 32 + (s_w & 1) < nkb ? sc_off + (uint32_t)((kt / 32) * 4) : W8_OOB;
            rsc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rss[s_op], (int)o, 0, 0));
        }
    };
    const int st_u = 2 * (tid & 3), st_sw = (ld_row >> 1) & 7;
    const int st_a0 = ld_row * 128 + 16 * (st_u ^ st_sw), st_a1 = ld_row * 128 + 16 * ((st_u + 1) ^ st_sw);
    auto store = [&](int buf) {
#pragma unroll
        for (int op = 0; op < 2; ++op) {
            const uint4 v = rt[op];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t h[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                h[2 * d] = op == 0 ? cvt2_f16<FA>(w[d], false) : cvt2_f16<FB>(w[d], false);
                h[2 * d + 1] = op == 0 ? cvt2_f16<FA>(w[d], true) : cvt2_f16<FB>(w[d], true);
            }
            *(uint4*)&sT[buf][op][st_a0] = make_uint4(h[0], h[1], h[2], h[3]);
            *(uint4*)&sT[buf][op][st_a1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
        sS[buf][s_op][s_w] = rsc;
    };

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int frow = lane & 15, g = lane >> 4, fsw = (frow >> 1) & 7;
    const int fa_off[2] = {(wm * WTM + frow) * 128 + 16 * (g ^ fsw), (wm * WTM + frow) * 128 + 16 * ((4 + g) ^ fsw)};
    const int fb_off[2] = {(wn * WTN + frow) * 128 + 16 * (g ^ fsw), (wn * WTN + frow) * 128 + 16 * ((4 + g) ^ fsw)};
    const int sal_off = (wm * WTM + 16 * (frow >> 2) + 4 * g + (frow & 3)) * 2, sb_off = (wn * WTN + frow) * 2;

    // K step t (LDS buffer BUF); MORE: tile t + 1 exists, so it is loaded during this step and
    // decoded into the other buffer after it.
    auto step = [&](int t, auto buf_c, auto more_c) {
        constexpr int BUF = decltype(buf_c)::value;
        constexpr bool MORE = decltype(more_c)::value;
        if constexpr (MORE) load((t + 1) * KS);
        f16x8 bf[TJ][2], af[TI][2];
        float2 sbv[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) bf[j][q] = *(const f16x8*)&sT[BUF][1][fb_off[q] + j * 16 * 128];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q) af[i][q] = *(const f16x8*)&sT[BUF][0][fa_off[q] + i * 16 * 128];
#pragma unroll
        for (int j = 0; j < TJ; ++j) sbv[j] = *(const float2*)&sS[BUF][1][sb_off + j * 32];
        const float2 sal = *(const float2*)&sS[BUF][0][sal_off];
        f32x4 p[2][2][TJ];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                p[0][q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[0][q], bf[j][q], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int cb = i & 1;
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    if (q == 0 && j == 0 && i + 2 < TI) {
#pragma unroll
                        for (int qq = 0; qq < 2; ++qq)
                            af[i + 2 < TI ? i + 2 : i][qq] = *(const f16x8*)&sT[BUF][0][fa_off[qq] + (i + 2) * 16 * 128];
                    }
                    if (i + 1 < TI)
                        p[cb ^ 1][q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i + 1 < TI ? i + 1 : i][q], bf[j][q],
                                                                               f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    const float sbq = q == 0 ? sbv[j].x : sbv[j].y;
                    float sc[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) sc[r] = w8_mul_bcast(q == 0 ? sal.x : sal.y, sbq, 4 * i + r);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(p[cb][q][j][r], sc[r], acc[i][j][r]);
                    // keep the multiply-adds in this group (the compiler would sink them to their
                    // next use, a step later)
#pragma unroll
                    for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(acc[i][j][r]));
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
        if constexpr (MORE) store(BUF ^ 1);
        __syncthreads();
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    load(0);
    store(0);
    __syncthreads();
    int t = 0;
    for (; t + 2 < ntile; t += 2) {
        step(t, B0{}, std::true_type{});
        step(t + 1, B1{}, std::true_type{});
    }
    if (t + 1 < ntile) {
        step(t, B0{}, std::true_type{});
        step(t + 1, B1{}, std::false_type{});
    } else {
        step(t, B0{}, std::false_type{});
    }
    w8_store<TI, TJ, WTM, WTN, false, W8_BLOCK>(acc, sa, sb, bias, c, M, N, m0, n0, wm, wn, lane);
}

// ---- native FP8 kernel: FP8 tiles in LDS, 128-byte rows; 16-byte chunk c of row r sits at
// chunk c ^ ((r >> 1) & 7) (16 consecutive rows reading one chunk hit 16 distinct bank groups).
// v_mfma*_16x16x128_f8f6f4 operand layout (measured): lane l holds row l & 15 with
// k = 16g .. 16g+15 in bytes 0..15 and k = 64 + 16g .. +15 in bytes 16..31 (g = l >> 4), and takes
// the scale of block b = k / 32 of that row from lane 16b + (l & 15).  So lane l reads chunks g and
// 4 + g and passes the scale byte of (row l & 15, block g).
// For FP32 block scales (four v_mfma_f32_16x16x32, lane k-slot 8g + 0..7 each), the 8-byte units
// of a row are stored transposed (unit k/8 = 4q + g at position 4g + q), so lane group g reads
// 32 contiguous bytes holding its 8 bytes of blocks q = 0..3.
template <int FA, int FB, bool UE8M0, int MODE>
struct W8MxCfg {
    static constexpr bool F32BLOCK = MODE == W8_BLOCK && !UE8M0;
    // FP32 block scales: fp32 multiply-adds on every 32-block partial need the accumulators in
    // VGPRs, so a 128 x 128 tile of 4 waves.  Row/column scales: 256 x 256 with 8 waves (2 x 4,
    // two per SIMD, 128 x 64 each), so one wave's LDS and load work overlaps the other's MFMAs
    // (1.8 PFLOP/s at 8192^3, against 1.6 with 4 waves).  UE8M0 block scales: the scaled MFMA
    // form needs far more registers than the unscaled one (the same kernel with the scaled form
    // and constant scales spills 136 VGPRs at 256 registers per wave), so 4 waves, one per SIMD,
    // with 512 registers each.
    static constexpr int BT = F32BLOCK ? 128 : 256;
    static constexpr int WM = 2, WN = (MODE == W8_ROWCOL) ? 4 : 2, NT = 64 * WM * WN;
};

template <int FA, int FB, bool UE8M0, int MODE>
__global__ __attribute__((amdgpu_flat_work_group_size(1, (W8MxCfg<FA, FB, UE8M0, MODE>::NT)))) void w8_mx_kernel(
    const uint8_t* __restrict__ a, const void* __restrict__ sa, const uint8_t* __restrict__ bt,
    const void* __restrict__ sb, const float* __restrict__ bias, float* __restrict__ c, int M, int N, int K) {
    using C = W8MxCfg<FA, FB, UE8M0, MODE>;
    constexpr int BT = C::BT, WM = C::WM, WN = C::WN, NT = C::NT;
    constexpr int WTM = BT / WM, WTN = BT / WN, TI = WTM / 16, TJ = WTN / 16;
    constexpr bool F32BLOCK = C::F32BLOCK, BLK = MODE == W8_BLOCK;
    constexpr int XA = FA == TFP8_E4M3FN ? 0 : 1, XB = FB == TFP8_E4M3FN ? 0 : 1;   // cbsz / blgp codes
    // UE8M0 scales stay bytes here (the instruction takes them raw): loaded below, not by W8Loader.
    using L = W8Loader<BT, false, F32BLOCK, NT>;
    constexpr int NS8 = 2 * BT / NT;   // UE8M0 scale words (4 blocks of one row) per thread per step
    static_assert(!(BLK && UE8M0) || (2 * BT) % NT == 0, "UE8M0 scale words fill whole thread sweeps");
    __shared__ __attribute__((aligned(16))) uint8_t sT[2][2][BT * 128];
    __shared__ __attribute__((aligned(16))) uint32_t sS[2][2][BLK ? BT * (F32BLOCK ? 4 : 1) : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int m0, n0;
    w8_tile(M, N, BT, m0, n0);
    L ld(a, sa, bt, sb, M, N, K, m0, n0);
    const int nkb = K / 32, ntile = (K + 127) / 128;

    // UE8M0 block scales: per step one word per row (bytes = blocks kb0 .. kb0+3).
    __amdgpu_buffer_rsrc_t rsu[2];
    uint32_t rsc8[NS8 > 0 ? NS8 : 1];
    if constexpr (BLK && UE8M0) {
        rsu[0] = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)sa + (size_t)m0 * nkb), (short)0,
                                                   (int)((uint32_t)min(BT, M - m0) * (uint32_t)nkb), (int)W8_FLAGS);
        rsu[1] = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)sb + (size_t)n0 * nkb), (short)0,
                                                   (int)((uint32_t)min(BT, N - n0) * (uint32_t)nkb), (int)W8_FLAGS);
    }
    // word w = wave * 64 + i * NT + lane of the 2 x BT step words: operand (w / BT) is wave-uniform
    auto s8_op = [&](int i) { return (wave * 64 + i * NT) / BT; };
    auto s8_row = [&](int i) { return (wave * 64 + i * NT) % BT + lane; };
    auto load = [&](int kt) {
        ld.load(kt, tid);
        if constexpr (BLK && UE8M0) {
            const int kb0 = kt / 32;
#pragma unroll
            for (int i = 0; i < NS8; ++i) {
                const int op = s8_op(i), row = s8_row(i);
                uint32_t v = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t o = kb0 + b < nkb ? (uint32_t)(row * nkb + kb0 + b) : W8_OOB;
                    v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rsu[op], (int)o, 0, 0) << (8 * b);
                }
                rsc8[i] = v;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int op = 0; op < 2; ++op)
#pragma unroll
            for (int i = 0; i < L::CH; ++i) {
                const int ch = tid + i * NT, row = ch >> 3, cc = ch & 7, sw = (row >> 1) & 7;
                uint8_t* base = &sT[buf][op][row * 128];
                const uint4 v = ld.rt[op][i];
                if constexpr (F32BLOCK) {
                    // units 2cc, 2cc+1 (q = cc >> 1, g = 2 (cc & 1) + 0/1) -> positions 4g + q
                    const int p0 = 8 * (cc & 1) + (cc >> 1), p1 = p0 + 4;
                    *(uint2*)(base + 16 * ((p0 >> 1) ^ sw) + 8 * (p0 & 1)) = make_uint2(v.x, v.y);
                    *(uint2*)(base + 16 * ((p1 >> 1) ^ sw) + 8 * (p1 & 1)) = make_uint2(v.z, v.w);
                } else {
                    *(uint4*)(base + 16 * (cc ^ sw)) = v;
                }
            }
        if constexpr (F32BLOCK) {
#pragma unroll
            for (int i = 0; i < L::NSW; ++i) {
                const int w = tid + i * NT;
                sS[buf][i * NT / (BT * 4)][w % (BT * 4)] = __float_as_uint(ld.rsc[i]);
            }
        } else if constexpr (BLK) {
#pragma unroll
            for (int i = 0; i < NS8; ++i) sS[buf][s8_op(i)][s8_row(i)] = rsc8[i];
        }
    };

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int frow = lane & 15, g = lane >> 4, sw = (frow >> 1) & 7;
    // this lane's two 16-byte chunks of a row: (g, 4 + g) for f8f6f4; (2g, 2g+1) for the transposed layout
    const int c0 = 16 * ((F32BLOCK ? 2 * g : g) ^ sw), c1 = 16 * ((F32BLOCK ? 2 * g + 1 : 4 + g) ^ sw);
    auto frag = [&](int buf, int op, int row) -> i32x8 {
        const uint8_t* base = &sT[buf][op][row * 128];
        const uint4 lo = *(const uint4*)(base + c0), hi = *(const uint4*)(base + c1);
        return i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    };

    load(0);
    store(0);
    __syncthreads();
    for (int t = 0; t < ntile; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntile) load((t + 1) * 128);
        if constexpr (F32BLOCK) {
            i32x8 bf[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) bf[j] = frag(buf, 1, wn * WTN + j * 16 + frow);
            float4 sbv[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) sbv[j] = *(const float4*)&sS[buf][1][(wn * WTN + j * 16 + frow) * 4];
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const i32x8 af = frag(buf, 0, wm * WTM + i * 16 + frow);
                float4 sav[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sav[r] = *(const float4*)&sS[buf][0][(wm * WTM + i * 16 + 4 * g + r) * 4];
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const long av = (long)(uint32_t)af[2 * q] | ((long)(uint32_t)af[2 * q + 1] << 32);
                        const long bv = (long)(uint32_t)bf[j][2 * q] | ((long)(uint32_t)bf[j][2 * q + 1] << 32);
                        const f32x4 p = w8_mma<FA, FB>(av, bv, f32x4{0.f, 0.f, 0.f, 0.f});
                        const float sbq = q == 0 ? sbv[j].x : q == 1 ? sbv[j].y : q == 2 ? sbv[j].z : sbv[j].w;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float saq = q == 0 ? sav[r].x : q == 1 ? sav[r].y : q == 2 ? sav[r].z : sav[r].w;
                            acc[i][j][r] = fmaf(p[r], saq * sbq, acc[i][j][r]);
                        }
                    }
            }
        } else {
            // With two waves per SIMD (256 registers per wave) the column tiles go in groups of
            // JH = 2: only two B fragments and one A fragment are live next to the accumulators,
            // and each A fragment is read from LDS TJ / JH times.
            constexpr int JH = NT == 512 && TJ >= 4 ? 2 : TJ;
#pragma unroll
            for (int jh = 0; jh < TJ; jh += JH) {
                i32x8 bf[JH];
                int sbs[JH];
#pragma unroll
                for (int j = 0; j < JH; ++j) {
                    bf[j] = frag(buf, 1, wn * WTN + (jh + j) * 16 + frow);
                    if constexpr (BLK) sbs[j] = (int)(sS[buf][1][wn * WTN + (jh + j) * 16 + frow] >> (8 * g));
                }
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const i32x8 af = frag(buf, 0, wm * WTM + i * 16 + frow);
                    if constexpr (BLK) {
                        const int sas = (int)(sS[buf][0][wm * WTM + i * 16 + frow] >> (8 * g));
#pragma unroll
                        for (int j = 0; j < JH; ++j)
                            acc[i][jh + j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                af, bf[j], acc[i][jh + j], XA, XB, 0, sas, 0, sbs[j]);
                    } else {
#pragma unroll
                        for (int j = 0; j < JH; ++j)
                            acc[i][jh + j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                af, bf[j], acc[i][jh + j], XA, XB, 0, 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);   // one A fragment live at a time
                }
            }
        }
        if (t + 1 < ntile) store(buf ^ 1);
        __syncthreads();
    }
    w8_store<TI, TJ, WTM, WTN, UE8M0, MODE>(acc, sa, sb, bias, c, M, N, m0, n0, wm, wn, lane);
}

// ---- exact kernel with scales folded into the decode: UE8M0 block scales and row/column scales.
// Codes are decoded to bf16 by v_cvt_scalef32_pk_bf16_{fp8,bf8}, whose scale operand carries an
// E8M0 exponent: with UE8M0 block scales the thread passes 2^(byte-127) (bits byte << 23), so the
// bf16 value is code * scale exactly (4 or 3 significant bits, and fp32's exponent range, fit bf16
// for every product above 2^-126 -- scales from the quantizer are >= 2^-40).  Then
// v_mfma_f32_16x16x32_bf16 accumulates in fp32 with exact products: C = sum_kb sum_k (A sa)(B sb),
// the reference's per-block sum with the scales moved inside, with no per-block multiply-add.
// Row/column scales decode with scale 1 and go to the epilogue.
template <int F>
__device__ __forceinline__ uint32_t w8_cvt_bf16(uint32_t w, float scale, bool hi) {
    bf16x2 v;
    if constexpr (F == TFP8_E4M3FN)
        v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, scale, true)
               : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, scale, false);
    else
        v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, scale, true)
               : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, scale, false);
    return __builtin_bit_cast(uint32_t, v);
}

// 256 x 256 tile, 8 waves of 128 x 64 (two per SIMD).  Each K step (64 wide) of A and Bt is loaded
// into registers one step ahead, decoded to bf16 with its block's E8M0 scale folded in and written
// to the other half of a double-buffered LDS pair (2 x 2 x 32 KB); the waves then read bf16
// fragments.  Every code is decoded once per block: decoding each wave's fragments right before
// its MFMAs instead decodes an A code in 4 waves and a Bt code in 2, and ran 10 % slower at 8192^3.
// LDS rows are 64 bf16 = 128 bytes; 16-byte chunk u of row r sits at u ^ ((r >> 1) & 7), so the
// 16 rows one fragment read touches land on distinct bank groups.
template <int FA, int FB, bool UE8M0, int MODE>
__global__ __launch_bounds__(512) void w8_bf16_kernel(const uint8_t* __restrict__ a, const void* __restrict__ sa,
                                                       const uint8_t* __restrict__ bt, const void* __restrict__ sb,
                                                       const float* __restrict__ bias, float* __restrict__ c, int M,
                                                       int N, int K) {
    constexpr int BT = 256, WM = 2, WN = 4, NT = 512, KT = 64;
    constexpr int WTM = BT / WM, WTN = BT / WN, TI = WTM / 16, TJ = WTN / 16;
    constexpr int CH = BT * (KT / 16) / NT;   // 16-code chunks per thread and operand
    constexpr bool BLK = MODE == W8_BLOCK;
    static_assert(!BLK || UE8M0, "FP32 block scales cannot be folded into the decode");
    __shared__ __attribute__((aligned(16))) uint8_t sT[2][2][BT * 128];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int m0, n0;
    w8_tile(M, N, BT, m0, n0);
    const int nkb = K / 32, ntile = (K + KT - 1) / KT;
    const uint32_t rows[2] = {(uint32_t)min(BT, M - m0), (uint32_t)min(BT, N - n0)};
    __amdgpu_buffer_rsrc_t rs[2], rss[2];
    rs[0] = __builtin_amdgcn_make_buffer_rsrc((void*)(a + (size_t)m0 * K), (short)0, (int)(rows[0] * (uint32_t)K),
                                              (int)W8_FLAGS);
    rs[1] = __builtin_amdgcn_make_buffer_rsrc((void*)(bt + (size_t)n0 * K), (short)0, (int)(rows[1] * (uint32_t)K),
                                              (int)W8_FLAGS);
    if constexpr (BLK) {
        rss[0] = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)sa + (size_t)m0 * nkb), (short)0,
                                                   (int)(rows[0] * (uint32_t)nkb), (int)W8_FLAGS);
        rss[1] = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)sb + (size_t)n0 * nkb), (short)0,
                                                   (int)(rows[1] * (uint32_t)nkb), (int)W8_FLAGS);
    }

    // Chunk ch = tid + i * NT of an operand: row ch >> 2, codes k = kt + 16 (ch & 3) .. +15, all in
    // scale block (kt + 16 (ch & 3)) / 32.  Past K (and past the rows of the block) the loads read
    // zeros; a zero scale byte decodes zero codes to zero.
    uint4 rt[2][CH];
    uint32_t rsb[2][CH];
    auto load = [&](int kt) {
#pragma unroll
        for (int op = 0; op < 2; ++op)
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int ch = tid + i * NT, row = ch >> 2, k = kt + 16 * (ch & 3);
                const uint32_t off = k < K ? (uint32_t)row * (uint32_t)K + (uint32_t)k : W8_OOB;
                rt[op][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs[op], (int)off, 0, 0));
                if constexpr (BLK) {
                    const uint32_t o = k < K ? (uint32_t)(row * nkb + k / 32) : W8_OOB;
                    rsb[op][i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rss[op], (int)o, 0, 0);
                }
            }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int op = 0; op < 2; ++op)
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int ch = tid + i * NT, row = ch >> 2, u = 2 * (ch & 3), sw = (row >> 1) & 7;
                const float s = BLK ? __uint_as_float(rsb[op][i] << 23) : 1.f;
                const uint4 v = rt[op][i];
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
                uint32_t h[8];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    h[2 * d] = op == 0 ? w8_cvt_bf16<FA>(w[d], s, false) : w8_cvt_bf16<FB>(w[d], s, false);
                    h[2 * d + 1] = op == 0 ? w8_cvt_bf16<FA>(w[d], s, true) : w8_cvt_bf16<FB>(w[d], s, true);
                }
                uint8_t* base = &sT[buf][op][row * 128];
                *(uint4*)(base + 16 * (u ^ sw)) = make_uint4(h[0], h[1], h[2], h[3]);
                *(uint4*)(base + 16 * ((u + 1) ^ sw)) = make_uint4(h[4], h[5], h[6], h[7]);
            }
    };

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Lane l of an MFMA for block q of the step reads row l & 15, k = 32q + 8 (l >> 4) .. +7:
    // logical chunk 4q + (l >> 4).
    const int frow = lane & 15, g = lane >> 4, fsw = (frow >> 1) & 7;
    auto frag = [&](int buf, int op, int row, int q) -> bf16x8 {
        return *(const bf16x8*)&sT[buf][op][row * 128 + 16 * ((4 * q + g) ^ fsw)];
    };

    // The loop keeps its conditional load and store: with the steady state split off branch-free
    // (as the f16 kernel does) this kernel ran 5 % slower (1285 vs 1219 us at 8192^3).
    load(0);
    store(0);
    __syncthreads();
    for (int t = 0; t < ntile; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntile) load((t + 1) * KT);
#pragma unroll
        for (int q = 0; q < KT / 32; ++q) {
            bf16x8 bd[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) bd[j] = frag(buf, 1, wn * WTN + j * 16 + frow, q);
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const bf16x8 ad = frag(buf, 0, wm * WTM + i * 16 + frow, q);
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ad, bd[j], acc[i][j], 0, 0, 0);
            }
        }
        if (t + 1 < ntile) store(buf ^ 1);
        __syncthreads();
    }
    w8_store<TI, TJ, WTM, WTN, UE8M0, MODE>(acc, sa, sb, bias, c, M, N, m0, n0, wm, wn, lane);
}

template <int FA, int FB, bool UE8M0, int MODE>
void w8_launch(bool native, const uint8_t* a, const void* sa, const uint8_t* bt, const void* sb, const float* bias,
               float* c, int M, int N, int K, hipStream_t s) {
    if (native) {
        using C = W8MxCfg<FA, FB, UE8M0, MODE>;
        const unsigned grid = (unsigned)(((M + C::BT - 1) / C::BT) * ((N + C::BT - 1) / C::BT));
        w8_mx_kernel<FA, FB, UE8M0, MODE><<<grid, C::NT, 0, s>>>(a, sa, bt, sb, bias, c, M, N, K);
        return;
    }
    if constexpr (MODE == W8_ROWCOL || UE8M0) {   // scales fold into the decode or the epilogue
        const unsigned grid = (unsigned)(((M + 255) / 256) * ((N + 255) / 256));
        w8_bf16_kernel<FA, FB, UE8M0, MODE><<<grid, 512, 0, s>>>(a, sa, bt, sb, bias, c, M, N, K);
    } else {                                       // FP32 block scales: per-block multiply-add
        const unsigned grid = (unsigned)(((M + 127) / 128) * ((N + 127) / 128));
        w8_f16_kernel<FA, FB><<<grid, 512, 0, s>>>(a, (const float*)sa, bt, (const float*)sb, bias, c, M, N, K);
    }
}

}  // namespace

extern "C" int tfp8_w8a8_quantize(const void* x, int x_dtype, int R, int K, int fmt, int ue8m0, uint8_t* q,
                                  void* scale, void* stream) {
    clear_error();
    if (R < 0 || K < 0 || !valid_fmt(fmt) || !valid_dtype(x_dtype))
        return fail(TFP8_ERR_ARG, "tfp8_w8a8_quantize: bad R/K/fmt/dtype");
    if (K % 32) return fail(TFP8_ERR_SHAPE, "tfp8_w8a8_quantize: K=%d must be a multiple of 32", K);
    if (R == 0 || K == 0) return 0;
    if (!x || !q || !scale) return fail(TFP8_ERR_ARG, "tfp8_w8a8_quantize: null pointer");
    if ((uintptr_t)q % 16) return fail(TFP8_ERR_ALIGN, "tfp8_w8a8_quantize: q must be 16-byte aligned");
    const int64_t blocks = (int64_t)R * (K / 32);
    const unsigned grid = (unsigned)((blocks + 255) / 256);
    hipStream_t s = (hipStream_t)stream;
    TFP8_DISPATCH_FMT(fmt, F, TFP8_DISPATCH_DT(x_dtype, D, {
        if (ue8m0) w8_quantize_kernel<F, D, true><<<grid, 256, 0, s>>>(x, R, K, q, scale);
        else w8_quantize_kernel<F, D, false><<<grid, 256, 0, s>>>(x, R, K, q, scale);
    }));
    return check_launch("tfp8_w8a8_quantize");
}

extern "C" int tfp8_w8a8_gemm(const uint8_t* a, int fmt_a, const void* sa, const uint8_t* bt, int fmt_b,
                              const void* sb, int ue8m0, int mode, int native_fp8, const float* bias, float* c, int M,
                              int N, int K, void* stream) {
    clear_error();
    if (M < 0 || N < 0 || K < 0 || !valid_fmt(fmt_a) || !valid_fmt(fmt_b) || (mode != W8_BLOCK && mode != W8_ROWCOL))
        return fail(TFP8_ERR_ARG, "tfp8_w8a8_gemm: bad M/N/K/format/mode");
    if (K % 32) return fail(TFP8_ERR_SHAPE, "tfp8_w8a8_gemm: K=%d must be a multiple of 32", K);
    if (M == 0 || N == 0) return 0;
    if (!a || !sa || !bt || !sb || !c) return fail(TFP8_ERR_ARG, "tfp8_w8a8_gemm: null pointer");
    if ((uintptr_t)a % 16 || (uintptr_t)bt % 16)
        return fail(TFP8_ERR_ALIGN, "tfp8_w8a8_gemm: A and Bt must be 16-byte aligned");
    if ((size_t)256 * K >= (1ull << 31)) return fail(TFP8_ERR_SHAPE, "tfp8_w8a8_gemm: K=%d too large", K);
    hipStream_t s = (hipStream_t)stream;
#define TFP8_W8(FA_, FB_)                                                                        \
    {                                                                                            \
        if (mode == W8_BLOCK) {                                                                  \
            if (ue8m0) w8_launch<FA_, FB_, true, W8_BLOCK>(native_fp8 != 0, a, sa, bt, sb, bias, c, M, N, K, s);   \
            else w8_launch<FA_, FB_, false, W8_BLOCK>(native_fp8 != 0, a, sa, bt, sb, bias, c, M, N, K, s);        \
        } else {                                                                                 \
            if (ue8m0) w8_launch<FA_, FB_, true, W8_ROWCOL>(native_fp8 != 0, a, sa, bt, sb, bias, c, M, N, K, s);  \
            else w8_launch<FA_, FB_, false, W8_ROWCOL>(native_fp8 != 0, a, sa, bt, sb, bias, c, M, N, K, s);       \
        }                                                                                        \
    }
    TFP8_DISPATCH_FMT(fmt_a, FA, TFP8_DISPATCH_FMT(fmt_b, FB, TFP8_W8(FA, FB)));
#undef TFP8_W8
    return check_launch("tfp8_w8a8_gemm");
}

}  // namespace tfp8
