// FP8-weight GEMM for many activation rows (M > 64) with one scale per weight row, on gfx950.
//
// y[m,n] = xs[m] * s[n] * sum_k x[m,k] * decode(w[n,k]) + bias[n]
// (reference gemm_w8a16, tfp8/csrc/tfp8_kernels.cu:271-411, per-channel / per-tensor case; the
// reference's chunked path, tfp8/linear.py:107-128, computes the same product).  Built around
// gfx950 measurements:
//   * buffer_load ... lds moves a K step's activation tile (f16/bf16, BM x 64) and raw FP8 weight
//     tile (BN x 64) straight into LDS, no VGPR staging and no ds_write; the steps form a ring of
//     S buffers (up to 160 KB), loads issued S-1 steps ahead, one barrier per K step;
//   * v_mfma_f32_32x32x16_{f16,bf16}; at M = 256 the 128 x 256 block tile is 8 waves of 64 x 64
//     (two per SIMD, so one wave's waits are covered by the other's MFMAs);
//   * ds_read_b128 moves about twice the bytes per clock of ds_read_b64, so a lane reads 16 codes
//     of a weight row at once.  Inside each 32-wide K window, lane half h (lane >> 5) holds
//     k = 16h .. 16h+15: codes 0-7 feed one MFMA and codes 8-15 the next, and the activation
//     fragments are read in the same K order, so every product x[m,k] * w[n,k] is formed exactly
//     once (only the fp32 summation order differs from the other GEMM kernels);
//   * fragments are read from LDS one whole K step before they are multiplied.
// Codes are decoded in registers with v_cvt_scalef32_pk_{f16,bf16}_{fp8,bf8} right before the
// MFMA; no decoded weight is ever written to LDS or HBM.  The scale, xs and bias are applied in
// the epilogue, or by the split-K reduction when K is split over gridDim.y.
#include <algorithm>
#include <type_traits>

#include "tfp8_common.h"

namespace tfp8 {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_void_t;

constexpr uint32_t GD_BUF_FLAGS = 0x00020000u;   // buffer resource word 3 (raw, 32-bit format)
constexpr int GD_BK = 64;                          // K step: 128-byte activation rows, 64-byte weight rows
constexpr int GD_LDS_MAX = 160 * 1024;             // LDS per workgroup on gfx950

template <typename T> struct GdOp;
template <> struct GdOp<_Float16> {
    typedef f16x8 V;
    static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, float s, bool hi) {
        f16x2 v;
        if constexpr (FMT == TFP8_E4M3FN) v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, false);
        else v = hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, false);
        return __builtin_bit_cast(uint32_t, v);
    }
};
template <> struct GdOp<__bf16> {
    typedef bf16x8 V;
    static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    template <int FMT> static __device__ __forceinline__ uint32_t cvt(uint32_t w, float s, bool hi) {
        bf16x2 v;
        if constexpr (FMT == TFP8_E4M3FN) v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, false);
        else v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, true) : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, false);
        return __builtin_bit_cast(uint32_t, v);
    }
};

// Scale handling: one scale per weight row (applied after the sum), UE8M0 K groups folded into
// the decode (the conversion multiplies by the scale's power of two, exact in bf16), or K groups
// (G % 64 == 0) applied to an fp32 partial sum at every group boundary (exact for any f32 scale).
enum { GD_CHANNEL = 0, GD_FOLD = 1, GD_PARTIAL = 2 };

// 8 codes (two dwords, k order) times the power of two of s -> one 16-bit MFMA operand.
template <typename T, int FMT>
__device__ __forceinline__ typename GdOp<T>::V gd_decode(uint32_t lo, uint32_t hi, float s) {
    uint4 u;
    u.x = GdOp<T>::template cvt<FMT>(lo, s, false);
    u.y = GdOp<T>::template cvt<FMT>(lo, s, true);
    u.z = GdOp<T>::template cvt<FMT>(hi, s, false);
    u.w = GdOp<T>::template cvt<FMT>(hi, s, true);
    return __builtin_bit_cast(typename GdOp<T>::V, u);
}

// One 16-byte-per-lane load into LDS: lane j's 16 bytes land at LDS byte lds + 16 j.  Written as
// inline assembly because the compiler, unable to tell which LDS bytes such a load writes, would
// otherwise wait for every load in flight before each LDS read; the kernel orders them itself
// (gd_wait_vm before the barrier that publishes a stage).
// The per-lane offset voff stays in one register for the whole K loop (the K position is the
// scalar soff), so no register a load still reads is ever overwritten.  m0 is a register the
// compiler reserves (hipcc warns about the clobber); these kernels give it no other use, which
// tests/test_isa_checks.py verifies on the generated code.
__device__ __forceinline__ void gd_load_lds(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory", "m0");
}

// Waits until at most N of this wave's load instructions are outstanding.
template <int N>
__device__ __forceinline__ void gd_wait_vm_const() {
    static_assert(N >= 0 && N <= 63, "vmcnt holds at most 63");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most `stages` stages of this wave's loads (L load instructions each) are
// outstanding, stages in 0..5.
template <int L>
__device__ __forceinline__ void gd_wait_vm(int stages) {
    static_assert(L >= 1 && 5 * L <= 63, "vmcnt holds at most 63");
    switch (stages) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * L) : "memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * L) : "memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * L) : "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * L) : "memory"); break;
    }
}

// Block tile BM x BN (BM = 32, 64 or 128 activation rows; BN = 128 or 256 weight rows), WM x WN
// waves, ring of S K steps.
template <typename T, int FMT, int BM, int BN, int WM, int WN, int S, int SMODE>
__global__ __launch_bounds__(64 * WM * WN) void gemm_direct_kernel(
    const T* __restrict__ x, const float* __restrict__ xs, const uint8_t* __restrict__ w,
    const void* __restrict__ ws, int sk, const float* __restrict__ bias, void* __restrict__ y, int ydt,
    int M, int N, int K, int G, float* __restrict__ part, int slice_len) {
    using Op = GdOp<T>;
    typedef typename Op::V V;
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN;     // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;     // 32 x 32 MFMA tiles per wave
    constexpr int ABYTES = BM * GD_BK * 2, STAGE = ABYTES + BN * GD_BK;
    constexpr int LA = BM / 8 / NW, LB = BN / 16 / NW;   // 1 KB loads per wave per stage
    static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile of whole 32x32 MFMA tiles");
    static_assert(LA >= 1 && LB >= 1 && LA * NW * 8 == BM && LB * NW * 16 == BN, "loads split evenly over waves");
    static_assert(S >= 3 && S <= 7 && S * STAGE <= GD_LDS_MAX, "ring of 3 to 7 stages in 160 KB of LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[S * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int l32 = lane & 31, h = lane >> 5;

    // XCD-aware tile order: consecutive ids land on one XCD and walk M first, so the blocks that
    // read one weight tile share an L2.
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN, nt = ntm * ntn;
    int id = blockIdx.x;
    if ((nt & 7) == 0) id = (blockIdx.x & 7) * (nt >> 3) + (blockIdx.x >> 3);
    const int m0 = (id % ntm) * BM, n0 = (id / ntm) * BN;
    const int kbeg = blockIdx.y * slice_len;
    const int nst = min(slice_len, K - kbeg) / GD_BK;   // whole K steps (K % 64 == 0, checked on the host)

    // Rows past M / N are out of range of these resources; whatever they leave in LDS only reaches
    // output rows / columns that are never stored.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(x + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * (uint32_t)K * 2u), (int)GD_BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(w + (size_t)n0 * K), (short)0, (int)((uint32_t)min(BN, N - n0) * (uint32_t)K), (int)GD_BUF_FLAGS);

    // K-group scales of the block's rows for the groups its K slice touches, staged in LDS once
    // (UE8M0 bytes for folding, f32 values for the partial sums).  Up to GD_SPT per thread (every
    // default shape), the loads go out together right before the first ring stages and are waited
    // for with them, so their latency overlaps the ring's; more than that, the staging loop runs
    // first, before any ring load is issued.
    extern __shared__ __attribute__((aligned(16))) uint8_t gd_scales[];
    const int gfirst = SMODE == GD_CHANNEL ? 0 : kbeg / G;
    const int nsg = SMODE == GD_CHANNEL ? 0 : (kbeg + nst * GD_BK - 1) / G - gfirst + 1;
    constexpr int GD_SPT = 16, TPR = NW * 64 / BN;   // scales per thread; threads per weight row
    static_assert(TPR >= 1 && TPR * BN == NW * 64, "whole threads per weight row");
    const bool scales_early = SMODE != GD_CHANNEL && nsg > GD_SPT * TPR;
    const int ng = SMODE == GD_CHANNEL ? 1 : K / G;
    if constexpr (SMODE != GD_CHANNEL) {
        if (scales_early) {
            for (int i = tid; i < BN * nsg; i += NW * 64) {
                const int r = i / nsg, n = min(n0 + r, N - 1);
                const size_t src = (size_t)n * ng + gfirst + (i - r * nsg);
                if constexpr (SMODE == GD_FOLD) gd_scales[i] = ((const uint8_t*)ws)[src];
                else ((float*)gd_scales)[i] = sk == TFP8_SCALE_UE8M0 ? ue8m0_to_f32(((const uint8_t*)ws)[src])
                                                                    : ((const float*)ws)[src];
            }
            __syncthreads();
        }
    }

    // LDS layouts (16-byte units): activation row r (128 B) keeps chunk c at c ^ ((r >> 1) & 7),
    // weight row r (64 B) keeps chunk c at c ^ ((r >> 2) & 3); both make the 16-row fragment
    // reads below conflict-free.  A load instruction fills 1 KB of LDS in lane order, so lane j of
    // instruction i fetches the global chunk that belongs at unit 64 i + j.
    uint32_t aoff[LA], boff[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int u = (wave * LA + i) * 64 + lane;
        const int ar = u >> 3, ac = (u & 7) ^ ((ar >> 1) & 7);
        aoff[i] = (uint32_t)ar * (uint32_t)K * 2u + (uint32_t)ac * 16u;
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
        const int u = (wave * LB + i) * 64 + lane;
        const int br = u >> 2, bc = (u & 3) ^ ((br >> 2) & 3);
        boff[i] = (uint32_t)br * (uint32_t)K + (uint32_t)bc * 16u;
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t)smem;
    // Loads K step st (K position kk) into the ring slot at LDS offset so.
    auto issue_at = [&](uint32_t so, uint32_t kk) {
        const uint32_t sa = lds0 + so;
#pragma unroll
        for (int i = 0; i < LA; ++i) gd_load_lds(ra, sa + (wave * LA + i) * 1024, aoff[i], kk * 2u);
#pragma unroll
        for (int i = 0; i < LB; ++i) gd_load_lds(rb, sa + ABYTES + (wave * LB + i) * 1024, boff[i], kk);
    };
    auto issue = [&](int st) { issue_at((uint32_t)(st % S) * STAGE, (uint32_t)(kbeg + st * GD_BK)); };

    // Fragment offsets inside a stage.  Window p (k = 32p .. 32p+31 of the step), half q:
    // activation chunk 4p + 2h + q of row wm*WTM + tm*32 + l32; weight chunk 2p + h of row
    // wn*WTN + tn*32 + l32 (16 codes: q = 0 uses the first 8, q = 1 the last 8).
    const int aswz = (l32 >> 1) & 7, bswz = (l32 >> 2) & 3;
    uint32_t a_rd[2][2], b_rd[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int q = 0; q < 2; ++q) a_rd[p][q] = (uint32_t)(wm * WTM + l32) * 128u + 16u * (uint32_t)((4 * p + 2 * h + q) ^ aswz);
        b_rd[p] = ABYTES + (uint32_t)(wn * WTN + l32) * 64u + 16u * (uint32_t)((2 * p + h) ^ bswz);
    }

    constexpr bool PART = SMODE == GD_PARTIAL;
    f32x16 acc[TM][TN], prt[PART ? TM : 1][PART ? TN : 1];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.f;
    if constexpr (PART) {
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) prt[a][b][i] = 0.f;
    }
    // This lane's column of tile tn inside the block, and its row of the staged scales.
    auto scale_row = [&](int tn) { return (wn * WTN + tn * 32 + l32) * nsg; };

    struct Frag {
        V a[TM][2];
        uint4 b[TN];
        uint32_t s[SMODE == GD_FOLD ? TN : 1];   // UE8M0 byte of the window's group, per tile; fix()
                                                 // turns it into the f32 scale's bits
    };
    // Reads window p of the stage at LDS offset so; g is the window's column of the staged scales
    // (G % 32 == 0: the window's 32 codes, both lane halves, lie in one group).
    auto read_at = [&](uint32_t so, int p, int g, Frag& f) {
        const uint8_t* base = smem + so;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) f.b[tn] = *(const uint4*)(base + b_rd[p] + tn * 2048);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int q = 0; q < 2; ++q) f.a[tm][q] = *(const V*)(base + a_rd[p][q] + tm * 4096);
        if constexpr (SMODE == GD_FOLD) {
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) f.s[tn] = gd_scales[scale_row(tn) + g];
        }
    };
    auto read = [&](int st, int p, Frag& f) {
        read_at((uint32_t)(st % S) * STAGE, p, SMODE == GD_FOLD ? (kbeg + st * GD_BK + 32 * p) / G - gfirst : 0, f);
    };
    // The scale bytes are converted at the end of the step that read them, after its MFMAs: the
    // wait for the byte then costs nothing, where converting it in read() would wait for the
    // fragment reads issued just before it.
    auto fix = [&](Frag& f) {
        if constexpr (SMODE == GD_FOLD) {
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) f.s[tn] = __float_as_uint(ue8m0_to_f32(f.s[tn]));
        }
    };
    auto mma = [&](const Frag& f) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const float sc = SMODE == GD_FOLD ? __uint_as_float(f.s[SMODE == GD_FOLD ? tn : 0]) : 1.f;
                const V bq = q ? gd_decode<T, FMT>(f.b[tn].z, f.b[tn].w, sc) : gd_decode<T, FMT>(f.b[tn].x, f.b[tn].y, sc);
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) {
                    if constexpr (PART) prt[tm][tn] = Op::mma(f.a[tm][q], bq, prt[tm][tn]);
                    else acc[tm][tn] = Op::mma(f.a[tm][q], bq, acc[tm][tn]);
                }
            }
    };
    // Partial sums: after the last K step of a group (G % 64 == 0) or of the slice, acc += prt * s.
    auto fold_group = [&](int t) {
        if constexpr (PART) {
            const int kn = kbeg + (t + 1) * GD_BK;
            if (kn % G == 0 || t == nst - 1) {
                const int g = (kn - 1) / G - gfirst;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const float sc = ((const float*)gd_scales)[scale_row(tn) + g];
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            acc[tm][tn][i] = fmaf(prt[tm][tn][i], sc, acc[tm][tn][i]);
                            prt[tm][tn][i] = 0.f;
                        }
                }
            }
        }
    };
    // Stage st is complete in LDS for every wave once each wave has waited for its own loads of it
    // (stages up to `last` have been issued; loads complete in order) and all have passed the barrier.
    auto sync_stage = [&](int st, int last) {
        gd_wait_vm<LA + LB>(last - st);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Pipeline: K steps 0..S-2 are loaded up front.  Step t+1 is published at the top of step t
    // (the same barrier retires step t-1's buffer, into which step t+S-1 is then issued), and both
    // K windows of step t+1 are read from LDS while step t multiplies: two register sets, swapped
    // by unrolling the loop by two.
    if constexpr (SMODE != GD_CHANNEL) {
        if (!scales_early) {
            // Thread tid stages entries j = q, q + TPR, ... (j < nsg) of row r.  The loads are inline
            // assembly like the ring's, so the compiler adds no wait of its own for them; the
            // explicit wait below retires them (they are older than every ring load) and the empty
            // asm statements keep every use of the values after it.
            const int r = tid / TPR, q = tid % TPR, n = min(n0 + r, N - 1);
            const bool f32s = SMODE == GD_PARTIAL && sk != TFP8_SCALE_UE8M0;
            const uint32_t esz = f32s ? 4u : 1u;
            const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
                (void*)ws, (short)0, (int)((uint32_t)N * (uint32_t)ng * esz), (int)GD_BUF_FLAGS);
            uint32_t sv[GD_SPT];
#pragma unroll
            for (int u = 0; u < GD_SPT; ++u) {
                const int j = min(q + TPR * u, nsg - 1);
                const uint32_t off = ((uint32_t)n * (uint32_t)ng + (uint32_t)(gfirst + j)) * esz;
                if (f32s) asm volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(sv[u]) : "v"(off), "s"(rsc) : "memory");
                else asm volatile("buffer_load_ubyte %0, %1, %2, 0 offen" : "=v"(sv[u]) : "v"(off), "s"(rsc) : "memory");
            }
            for (int st = 0; st < S - 1 && st < nst; ++st) issue(st);
            gd_wait_vm<LA + LB>(min(S - 1, nst));
#pragma unroll
            for (int u = 0; u < GD_SPT; ++u) {
                asm volatile("" : "+v"(sv[u]));
                const int j = q + TPR * u;
                if (j < nsg) {
                    if constexpr (SMODE == GD_FOLD) gd_scales[r * nsg + j] = (uint8_t)sv[u];
                    else ((float*)gd_scales)[r * nsg + j] = f32s ? __builtin_bit_cast(float, sv[u]) : ue8m0_to_f32(sv[u]);
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // published by sync_stage's barrier
        } else {
            for (int st = 0; st < S - 1 && st < nst; ++st) issue(st);
        }
    } else {
        for (int st = 0; st < S - 1 && st < nst; ++st) issue(st);
    }
    Frag f0, f1, g0, g1;
    sync_stage(0, min(nst - 1, S - 2));
    read(0, 0, f0);
    read(0, 1, f1);
    fix(f0);
    fix(f1);
    auto step = [&](int t, Frag& c0, Frag& c1, Frag& n0, Frag& n1) {
        const bool more = t + 1 < nst;
        if (more) sync_stage(t + 1, min(nst - 1, t + S - 2));
        if (t + S - 1 < nst) issue(t + S - 1);
        if (more) read(t + 1, 0, n0);
        mma(c0);
        if (more) read(t + 1, 1, n1);
        mma(c1);
        fold_group(t);
        if (more) {
            fix(n0);
            fix(n1);
        }
    };
    // Steady state, t + S - 1 < nst: every step issues a stage and reads the next fragments, so the
    // body has no branches and the wait counts are constants.  (With the conditional form above in
    // the loop, the compiler's wait counts at the merge points had to cover the LDS reads just
    // issued for the next step: lgkmcnt(0) before the last MFMAs of every step.)  The scheduling
    // barriers keep each window's reads ahead of the multiplies that overlap them.
    // The steady state carries its ring positions and scale column from step to step (a division
    // or remainder by a run-time G, or by a ring depth that is no power of two, costs a dozen scalar
    // instructions per use): rso / lso are the LDS offsets of the stages read and loaded next
    // (t + 1 and t + S - 1), lk the K position of the latter, and gq / gr the staged-scale column of
    // the next window to read and its position among the G / 32 windows of its group.
    constexpr uint32_t RING = (uint32_t)S * STAGE;
    uint32_t rso = (uint32_t)(1 % S) * STAGE, lso = (uint32_t)((S - 1) % S) * STAGE;
    uint32_t lk = (uint32_t)(kbeg + (S - 1) * GD_BK);
    const int wpg = SMODE == GD_FOLD ? G / 32 : 1;
    int gq = 0, gr = 0;
    if constexpr (SMODE == GD_FOLD) {
        const int w = kbeg / 32 + 2;                  // first window of step 1
        gq = w / wpg - gfirst;
        gr = w % wpg;
    }
    auto next_window = [&]() {
        if constexpr (SMODE == GD_FOLD) {
            const bool wrap = ++gr == wpg;
            gq += wrap ? 1 : 0;
            gr = wrap ? 0 : gr;
        }
    };
    auto step_full = [&](int t, Frag& c0, Frag& c1, Frag& n0, Frag& n1) {
        gd_wait_vm_const<(LA + LB) * (S - 3)>();     // stage t + 1 done; t + 2 .. t + S - 2 may be in flight
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_at(lso, lk);
        read_at(rso, 0, gq, n0);
        next_window();
        __builtin_amdgcn_sched_barrier(0);
        mma(c0);
        read_at(rso, 1, gq, n1);
        next_window();
        __builtin_amdgcn_sched_barrier(0);
        mma(c1);
        fold_group(t);
        fix(n0);
        fix(n1);
        if constexpr ((RING & (RING - 1)) == 0) {
            rso = (rso + STAGE) & (RING - 1);
            lso = (lso + STAGE) & (RING - 1);
        } else {
            rso = rso + STAGE == RING ? 0u : rso + STAGE;
            lso = lso + STAGE == RING ? 0u : lso + STAGE;
        }
        lk += GD_BK;
    };
    int t = 0;
    for (; t + 1 < nst - (S - 1); t += 2) {
        step_full(t, f0, f1, g0, g1);
        step_full(t + 1, g0, g1, f0, f1);
    }
    for (; t + 1 < nst; t += 2) {
        step(t, f0, f1, g0, g1);
        step(t + 1, g0, g1, f0, f1);
    }
    if (t < nst) step(t, f0, f1, g0, g1);

    // Epilogue.  32x32 MFMA output layout: lane l holds column l & 31 and rows
    // 8 (i >> 2) + 4 (l >> 5) + (i & 3) of accumulator element i.
    const int rbase = m0 + wm * WTM + 4 * h;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const int col = n0 + wn * WTN + tn * 32 + l32;
        if (col >= N) continue;
        if (part) {
            float* pp = part + (size_t)blockIdx.y * M * N;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = rbase + tm * 32 + 8 * (i >> 2) + (i & 3);
                    if (row < M) pp[(size_t)row * N + col] = acc[tm][tn][i];
                }
        } else {
            const float cs = SMODE != GD_CHANNEL          ? 1.f
                             : sk == TFP8_SCALE_UE8M0 ? load_scale<TFP8_SCALE_UE8M0>(ws, (size_t)col)
                                                      : load_scale<TFP8_SCALE_F32>(ws, (size_t)col);
            const float bv = bias ? bias[col] : 0.f;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = rbase + tm * 32 + 8 * (i >> 2) + (i & 3);
                    if (row < M) {
                        const float v = acc[tm][tn][i] * cs;
                        store_elem(y, (size_t)row * N + col, ydt, xs ? fmaf(v, xs[row], bv) : v + bv);
                    }
                }
        }
    }
}

}  // namespace

namespace {

// Launch configurations: block tile, wave grid, ring depth.
struct GdCfg {
    int bm, bn, wm, wn, stages;
};
constexpr GdCfg GD_CFGS[] = {
    {128, 256, 2, 4, 4},   // 0: M > 128 (C3 M=256), 8 waves of 64 x 64
    {128, 256, 2, 2, 4},   // 1: 4 waves of 64 x 128
    {128, 256, 2, 4, 3},   // 2
    {128, 256, 2, 4, 5},   // 3
    {64, 256, 2, 4, 6},    // 4: M <= 64, 8 waves of 32 x 64
    {32, 256, 1, 4, 7},    // 5: M <= 32, 4 waves of 32 x 64
    {128, 128, 2, 4, 6},   // 6: 8 waves of 64 x 32
    {64, 128, 2, 2, 5},    // 7: 4 waves of 32 x 64 (5 stages: 24.7 vs 25.7 us with 7 at C3 M=64)
};
constexpr int GD_NCFG = (int)(sizeof(GD_CFGS) / sizeof(GD_CFGS[0]));

// Smallest M this kernel takes; the weight-streaming kernel serves fewer rows.  Same-box sweep on
// MI355X at K = N = 8192, per-channel scales (us, weight-streaming vs this kernel's default
// configuration): M=24 20.2 vs 22.5, M=32 20.9 vs 23.4, M=48 25.3 vs 24.9, M=64 27.6 vs 25.4
// (64 x 128, 7 stages; 24.7 with the 5 stages now used); M=128 43.4 vs 33.3 (128 x 128, 6 stages); M=256 56.1 (LDS-tiled) vs 51
// (128 x 256, 4 stages).
int gd_min_m() { return tune(TUNE_GEMM_DIRECT_MIN_M); }

// Split of K for a tile grid: slices of whole 64-wide steps until the grid has a block per CU,
// slices of at least 1024.
int gd_slices(long tiles, int K) {
    int s = 1;
    while (tiles * s < 256 && s < 8 && K / (s * 2) >= 1024) s *= 2;
    return s;
}

// Above 128 rows the 128 x 256 tile, or 128 x 128 where the larger tile's grid has no more blocks
// than half the CUs (the C5 prefill, M=512: N=K=2048 20.4 -> 16.5 us, N=2048 K=5632 29.1 -> 24.5;
// with more blocks it loses: N=5632 K=2048 28.0 -> 33.5, M=4096 N=K=2048 48.6 -> 62.1).
GdCfg gd_cfg(int M, int N, int K) {
    int c = M > 128 ? 0 : M > 64 ? 6 : M > 32 ? 7 : 5;
    if (c == 0) {
        const long tiles = (long)((M + 127) / 128) * ((N + 255) / 256);
        if (tiles * gd_slices(tiles, K) <= 128) c = 6;
    }
    const int f = tune(TUNE_GEMM_DCFG);   // knob TFP8_GEMM_DCFG: index into GD_CFGS
    if (f >= 0 && f < GD_NCFG) c = f;
    return GD_CFGS[c];
}

}  // namespace

// Scale mode for (G, scale kind, activation dtype), or -1 where this kernel does not apply.
static int gd_mode(int K, int G, int ws_kind, int x16_dtype) {
    if (G == K) return GD_CHANNEL;
    if (ws_kind == TFP8_SCALE_UE8M0 && x16_dtype == TFP8_BF16 && G % 32 == 0) return GD_FOLD;
    if (G % 64 == 0) return GD_PARTIAL;
    return -1;
}

// Split of K: slices of whole 64-wide steps until the grid has a block per CU, slices of at least
// 1024.  Depends on the shape only (the workspace is sized from it).
static bool gd_split(int M, int N, int K, int* slices, int* slice_len) {
    if (K % GD_BK != 0 || M < gd_min_m() || !tune(TUNE_GEMM_DIRECT)) return false;
    const GdCfg c = gd_cfg(M, N, K);
    if ((long)c.bn * K >= (1L << 31) || (long)c.bm * K * 2 >= (1L << 31)) return false;
    const long tiles = (long)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    int s = gd_slices(tiles, K);
    const int fs = tune(TUNE_GEMM_SPLITK);
    if (fs > 0) s = std::min(fs, 8);
    int len = ((K + s - 1) / s + GD_BK - 1) / GD_BK * GD_BK;
    s = (K + len - 1) / len;
    *slices = s;
    *slice_len = s > 1 ? len : K;
    return true;
}

// Whether this kernel takes the GEMM, with its split of K, scale mode and dynamic LDS (the staged
// K-group scales of a block: they and the ring must fit the 160 KB of a workgroup; K-group modes
// exist for the default tiles only).
static bool gd_plan(int M, int N, int K, int G, int ws_kind, int x16_dtype, int* slices, int* slice_len, int* mode,
                    size_t* dyn) {
    const int md = gd_mode(K, G, ws_kind, x16_dtype);
    if (md < 0 || !gd_split(M, N, K, slices, slice_len)) return false;
    const GdCfg c = gd_cfg(M, N, K);
    *mode = md;
    *dyn = 0;
    if (md != GD_CHANNEL) {
        const bool dflt = (c.bm == 128 && c.bn == 256 && c.wm == 2 && c.wn == 4 && c.stages == 4) ||
                          (c.bm == 128 && c.bn == 128 && c.wm == 2 && c.wn == 4 && c.stages == 6);
        if (!dflt) return false;
        if ((size_t)N * (size_t)(K / G) * 4 >= (1ull << 31)) return false;   // scale buffer resource range
        const size_t groups = (size_t)(*slice_len / G + 2);   // groups one slice can touch
        *dyn = (c.bn * groups * (md == GD_FOLD ? 1 : 4) + 15) / 16 * 16;
    }
    const size_t ring = (size_t)c.stages * (c.bm * GD_BK * 2 + c.bn * GD_BK);
    return ring + *dyn <= (size_t)GD_LDS_MAX;
}

size_t gemm_direct_partial_bytes(int M, int N, int K) {
    int s, len;
    if (!gd_split(M, N, K, &s, &len)) return 0;
    return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

void splitk_reduce_launch(const float* part, int S, int M, int N, const void* ws, int sk, int colscale, const float* xs,
                          const float* bias, void* y, int ydt, int xcw, hipStream_t s);
int gemm_xcd_cols(int ntm, int ntn, int bn);

template <typename T, int FMT, int SMODE>
static void gd_launch(int slices, int slice_len, size_t dyn, const void* x, const float* xs, const uint8_t* w,
                      const void* ws, int sk, const float* bias, void* y, int ydt, int M, int N, int K, int G,
                      float* part, hipStream_t s) {
    const GdCfg c = gd_cfg(M, N, K);
    const dim3 grid(((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn), slices);
#define GD_K(BM_, BN_, WM_, WN_, S_)                                                                           \
    if (c.bm == BM_ && c.bn == BN_ && c.wm == WM_ && c.wn == WN_ && c.stages == S_) {                          \
        gemm_direct_kernel<T, FMT, BM_, BN_, WM_, WN_, S_, SMODE><<<grid, 64 * WM_ * WN_, dyn, s>>>(           \
            (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, part, slice_len);                            \
        return;                                                                                                \
    }
    GD_K(128, 256, 2, 4, 4)
    GD_K(128, 128, 2, 4, 6)
    if constexpr (SMODE == GD_CHANNEL) {
        GD_K(128, 256, 2, 2, 4)
        GD_K(128, 256, 2, 4, 3)
        GD_K(128, 256, 2, 4, 5)
        GD_K(64, 256, 2, 4, 6)
        GD_K(32, 256, 1, 4, 7)
        GD_K(64, 128, 2, 2, 5)
    }
#undef GD_K
}

template <typename T, int FMT>
static void gd_launch_mode(int mode, int slices, int slice_len, size_t dyn, const void* x, const float* xs,
                           const uint8_t* w, const void* ws, int sk, const float* bias, void* y, int ydt, int M, int N,
                           int K, int G, float* part, hipStream_t s) {
    if (mode == GD_PARTIAL)
        gd_launch<T, FMT, GD_PARTIAL>(slices, slice_len, dyn, x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, part, s);
    else if (mode == GD_FOLD) {
        if constexpr (std::is_same<T, __bf16>::value)
            gd_launch<T, FMT, GD_FOLD>(slices, slice_len, dyn, x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, part, s);
    } else
        gd_launch<T, FMT, GD_CHANNEL>(slices, slice_len, dyn, x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, part, s);
}

// Runs this GEMM if it takes the shape; returns NOT_TAKEN if it did not (caller falls back), 0 or an
// error code otherwise.  x16 is f16/bf16 [M,K]; partial is the caller's workspace, at least
// gemm_direct_partial_bytes(M, N, K) bytes.
int run_gemm_direct(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
                    const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype,
                    float* partial, hipStream_t s) {
    int slices, slice_len, mode;
    size_t dyn;
    if (!gd_plan(M, N, K, G, ws_kind, x16_dtype, &slices, &slice_len, &mode, &dyn)) return NOT_TAKEN;
    float* part = slices > 1 ? partial : nullptr;
    if (x16_dtype == TFP8_BF16) {
        TFP8_DISPATCH_FMT(fmt, F, gd_launch_mode<__bf16, F>(mode, slices, slice_len, dyn, x16, xs, w, ws, ws_kind,
                                                            bias, y, y_dtype, M, N, K, G, part, s));
    } else {
        TFP8_DISPATCH_FMT(fmt, F, gd_launch_mode<_Float16, F>(mode, slices, slice_len, dyn, x16, xs, w, ws, ws_kind,
                                                              bias, y, y_dtype, M, N, K, G, part, s));
    }
    int rc = check_launch("tfp8_gemm (direct)");
    if (rc || slices <= 1) return rc;
    const GdCfg c = gd_cfg(M, N, K);
    const int ntm = (M + c.bm - 1) / c.bm, ntn = (N + c.bn - 1) / c.bn;
    const int xcw = (ntm * ntn) % 8 == 0 ? gemm_xcd_cols(ntm, ntn, c.bn) : 0;
    splitk_reduce_launch(part, slices, M, N, ws, ws_kind, mode == GD_CHANNEL ? 1 : 0, xs, bias, y, y_dtype, xcw, s);
    return check_launch("tfp8_gemm (direct) splitk reduce");
}

}  // namespace tfp8
