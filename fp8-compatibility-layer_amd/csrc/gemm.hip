// LDS-tiled FP8-weight GEMM on gfx950 MFMA (M > 8 rows).
//
// y[m,n] = xs[m] * sum_g s(n,g) * sum_{k in g} x[m,k] * decode(w[n,k]) + bias[n]
// (reference gemm_w8a16, tfp8/csrc/tfp8_kernels.cu:271-411), built for CDNA4:
//   * block tile BM x BN x BK, WM x WN waves (8 for the large tiles: two waves per SIMD keep the
//     matrix cores fed, one cannot), wave tile (BM/WM) x (BN/WN) made of 16x16 outputs of
//     v_mfma_f32_16x16x32_{f16,bf16} (fp32 accumulation);
//   * per K tile the activation tile (f16/bf16) and the raw FP8 weight tile (1 byte per element,
//     half the LDS footprint of a decoded tile) are loaded with unconditional buffer loads
//     (rows past M/N and k past the slice read zeros) two tiles ahead into registers, then
//     written to a double-buffered LDS pair; each wave reads its 8-byte B fragments from LDS
//     and decodes them in registers with v_cvt_scalef32_pk_{f16,bf16}_{fp8,bf8} right before
//     the MFMA, so the weight is never written back decoded, to LDS or to HBM;
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

constexpr uint32_t GEMM_BUF_FLAGS = 0x00020000u;   // buffer resource word 3 (raw, 32-bit format)
constexpr uint32_t GEMM_OOB = 0x80000000u;         // a byte offset past every resource used here

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

__device__ __forceinline__ uint4 gload16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0));
}

template <typename T, int FMT, int BM, int BN, int WM, int WN, int BK, bool GROUPED>
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
    static_assert(BK % 32 == 0, "K tile is whole MFMA steps");
    // Activation tile rows are BK 16-bit values (128 or 256 bytes), unpadded; 16-byte chunk c of
    // row r sits at chunk c ^ swz(r).  Measured with the LDS bank-conflict counter: a 16-byte row
    // pad (272-byte rows) costs one extra cycle in every 16-lane pass of the fragment reads, while
    // this XOR layout is conflict-free for both the reads (16 rows, one chunk each) and the tile
    // writes (16 lanes per 256-byte row).
    constexpr int AROW = BK * 2;
    constexpr int BROW = BK + 16;
    constexpr int A_CPR = BK / 8, B_CPR = BK / 16;  // 16-byte chunks per tile row
    static_assert(A_CPR == 8 || A_CPR == 16, "A tile rows of 128 or 256 bytes");
    // 256-byte rows: 16 chunks, XOR with row & 15.  128-byte rows: 8 chunks, XOR with
    // (row >> 1) & 7, so rows r and r + 1 (same chunk index, other half of the banks) and r + 8 differ.
    auto aswz = [](int row) { return A_CPR == 16 ? (row & 15) : ((row >> 1) & 7); };
    constexpr int A_CHUNKS = BM * A_CPR, B_CHUNKS = BN * B_CPR;
    constexpr int CA = (A_CHUNKS + NT - 1) / NT;
    constexpr int CB = (B_CHUNKS + NT - 1) / NT;

    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * AROW];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][BN * BROW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // XCD-aware tile order: consecutive ids land on one XCD, and consecutive ids walk M first,
    // so blocks that read the same weight tile share an L2.
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN, nt = ntm * ntn;
    int id = blockIdx.x;
    if ((nt & 7) == 0) id = (blockIdx.x & 7) * (nt >> 3) + (blockIdx.x >> 3);
    const int m0 = (id % ntm) * BM, n0 = (id / ntm) * BN;

    const int kbeg = blockIdx.y * slice_len;
    const int kend = min(K, kbeg + slice_len);

    // One buffer resource per operand over this block's rows: rows past M / N are out of range
    // and read as zeros, so every load below is unconditional.
    const __amdgpu_buffer_rsrc_t ra_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(x + (size_t)m0 * K), (short)0, (int)((uint32_t)min(BM, M - m0) * (uint32_t)K * 2u), (int)GEMM_BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rb_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(w + (size_t)n0 * K), (short)0, (int)((uint32_t)min(BN, N - n0) * (uint32_t)K), (int)GEMM_BUF_FLAGS);

    // Per-lane chunk coordinates (fixed over the K loop).
    uint32_t a_row_off[CA], b_row_off[CB];
    int a_col[CA], b_col[CB];
#pragma unroll
    for (int i = 0; i < CA; ++i) {
        const int c = tid + i * NT;
        const int row = c / A_CPR;
        a_col[i] = (c % A_CPR) * 8;
        a_row_off[i] = c < A_CHUNKS ? (uint32_t)row * (uint32_t)K * 2u : GEMM_OOB;
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
        const int c = tid + i * NT;
        const int row = c / B_CPR;
        b_col[i] = (c % B_CPR) * 16;
        b_row_off[i] = c < B_CHUNKS ? (uint32_t)row * (uint32_t)K : GEMM_OOB;
    }

    uint4 ra[2][CA], rb[2][CB];
    // Global -> registers for the K tile at kt (k >= kend reads zeros).
    auto issue = [&](int slot, int kt) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int gk = kt + a_col[i];
            const uint32_t off = gk < kend ? a_row_off[i] + (uint32_t)gk * 2u : GEMM_OOB;
            ra[slot][i] = gload16(ra_rsrc, off);
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int gk = kt + b_col[i];
            const uint32_t off = gk < kend ? b_row_off[i] + (uint32_t)gk : GEMM_OOB;
            rb[slot][i] = gload16(rb_rsrc, off);
        }
    };
    auto commit = [&](int slot, int buf) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * NT;
            if (A_CHUNKS % NT == 0 || c < A_CHUNKS)
                *(uint4*)&sA[buf][(c / A_CPR) * AROW + (((c % A_CPR) ^ aswz(c / A_CPR)) * 16)] = ra[slot][i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = tid + i * NT;
            if (B_CHUNKS % NT == 0 || c < B_CHUNKS)
                *(uint4*)&sB[buf][(c / B_CPR) * BROW + (c % B_CPR) * 16] = rb[slot][i];
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

    // One K tile from LDS buffer `buf`.  The fragments of MFMA step ks+1 are read while step ks
    // multiplies, and the B operands of step ks+1 are decoded between the MFMAs of step ks
    // (one conversion in each MFMA's shadow), so neither LDS latency nor the decode leaves the
    // matrix core idle; the two waves of a SIMD run in phase after each barrier, so the
    // interleave has to happen inside the wave.
    auto compute = [&](int buf, int kt) {
        uint2 braw[2][TN];
        V araw[2][TM];
        V bf[2][TN];
        auto fetch = [&](int slot, int ks) {
#pragma unroll
            for (int b = 0; b < TN; ++b)
                braw[slot][b] = *(const uint2*)&sB[buf][(brow + b * 16) * BROW + ks * 32 + kq];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                araw[slot][a] = *(const V*)&sA[buf][(arow + a * 16) * AROW + (((ks * 32 + kq) / 8) ^ aswz(arow)) * 16];
        };
        auto decode = [&](int slot) {
#pragma unroll
            for (int b = 0; b < TN; ++b) bf[slot][b] = decode_frag<T, FMT>(braw[slot][b]);
        };
        fetch(0, 0);
        if (BK / 32 > 1) fetch(1, 1);
        decode(0);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int cur = ks & 1;
            __builtin_amdgcn_sched_barrier(0);
            // Steps past the slice end multiply the zeros their loads returned, so no step needs
            // a guard; an extra fold there adds prt = 0 (or NaN where a non-finite scale already
            // makes the column NaN).
            const int kk = kt + ks * 32;
            // MFMAs of this step in program order, each followed by its share of the next step's
            // conversions (none after the first two: their LDS reads may still be in flight);
            // sched_barrier(0) after each pair keeps the order.
            constexpr int NM = TM * TN, NC = 4 * TN;
            constexpr int LEAD = NM > 2 ? 2 : 0;
            constexpr int PER = NM > LEAD ? (NC + NM - LEAD - 1) / (NM - LEAD) : NC;
            const bool dec = ks + 1 < BK / 32;
            uint32_t nb[TN][4];
#pragma unroll
            for (int i = 0; i < NM; ++i) {
                const int a = i / TN, b = i % TN;
                if constexpr (GROUPED) prt[a][b] = Op::run(araw[cur][a], bf[cur][b], prt[a][b]);
                else acc[a][b] = Op::run(araw[cur][a], bf[cur][b], acc[a][b]);
                if (dec && i >= LEAD) {
#pragma unroll
                    for (int j = (i - LEAD) * PER; j < (i - LEAD + 1) * PER && j < NC; ++j) {
                        const int fb = j / 4, wd = j % 4;
                        const uint32_t src = (wd < 2) ? braw[cur ^ 1][fb].x : braw[cur ^ 1][fb].y;
                        nb[fb][wd] = Op::template cvt<FMT>(src, (wd & 1) != 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (dec) {
#pragma unroll
                for (int fb = 0; fb < TN; ++fb)
                    bf[cur ^ 1][fb] = __builtin_bit_cast(V, make_uint4(nb[fb][0], nb[fb][1], nb[fb][2], nb[fb][3]));
            }
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 2 < BK / 32) fetch(cur, ks + 2);   // this step's slot is free again
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
    };

    // Pipeline: LDS double buffer, and the global loads of a tile are issued two tiles ahead of
    // its use (register slots 0/1), so one full tile of MFMA work covers each load's latency.
    // Loads past the slice's end read zeros and are never consumed.
    // The loop runs whole pairs of tiles and an odd last tile is handled after it: a break in
    // the middle of the pair would merge a path with slot-0 loads still in flight into the
    // loop head, and the compiler would then drain every load there on every iteration.
    const int ntiles = (kend - kbeg + BK - 1) / BK;
    issue(0, kbeg);
    issue(1, kbeg + BK);
    commit(0, 0);
    __syncthreads();
    // sched_barrier(0) keeps each phase in place: otherwise the scheduler hoists the LDS writes
    // of the other buffer above the MFMA work (nothing orders them), which makes the wave wait
    // for the newest loads at the top of every half-iteration.
    int t = 0;
    for (; t + 1 < ntiles; t += 2) {
        issue(0, kbeg + (t + 2) * BK);
        __builtin_amdgcn_sched_barrier(0);
        compute(0, kbeg + t * BK);
        __builtin_amdgcn_sched_barrier(0);
        commit(1, 1);
        __syncthreads();
        issue(1, kbeg + (t + 3) * BK);
        __builtin_amdgcn_sched_barrier(0);
        compute(1, kbeg + (t + 1) * BK);
        __builtin_amdgcn_sched_barrier(0);
        commit(0, 0);
        __syncthreads();
    }
    if (t < ntiles) compute(0, kbeg + t * BK);

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

// Split-K epilogue: y = (sum_s part[s]) * colscale * xs + bias, slices added in order.
// Fast form: 8 consecutive columns per thread, every slice's loads issued before the first add,
// one 16-byte store per thread (N % 8 == 0, y 16-byte aligned, at most 8 slices); generic form:
// one column per thread.
// xcw > 0: the GEMM wrote output columns [x * xcw, (x + 1) * xcw) from XCD x (its blocks go
// round-robin over the 8 XCDs), and this kernel's blocks b with b % 8 == x (the same XCD) reduce
// exactly those columns, so they read partials their own L2 may still hold (C3 M=256: 9.7 ->
// 9.2 us); gridDim.x is then a multiple of 8.
template <int YDT, int SK>
__global__ __launch_bounds__(256) void splitk_reduce8_kernel(const float* __restrict__ part, int S, int M, int N,
                                                             const void* __restrict__ ws, int colscale,
                                                             const float* __restrict__ xs,
                                                             const float* __restrict__ bias, void* __restrict__ y,
                                                             int xcw) {
    const int64_t total = (int64_t)M * N;
    const int nv = N / 8;
    int cbase = 0, cv = nv;                         // column groups of 8 this block's XCD reduces
    int64_t it0 = (int64_t)blockIdx.x * 256 + threadIdx.x, step = (int64_t)gridDim.x * 256;
    if (xcw > 0) {
        cbase = (int)(blockIdx.x & 7) * (xcw / 8);
        cv = max(0, min(nv - cbase, xcw / 8));
        it0 = (int64_t)(blockIdx.x >> 3) * 256 + threadIdx.x;
        step = (int64_t)(gridDim.x >> 3) * 256;
    }
    const int64_t items = (int64_t)M * cv;
    for (int64_t it = it0; it < items; it += step) {
        const int row = (int)(it / cv), col = (cbase + (int)(it - (int64_t)row * cv)) * 8;
        const size_t i = (size_t)row * N + col;
        float4 lo[8], hi[8];
#pragma unroll
        for (int s = 0; s < 8; ++s)
            if (s < S) {
                lo[s] = *(const float4*)(part + (size_t)s * total + i);
                hi[s] = *(const float4*)(part + (size_t)s * total + i + 4);
            }
        float v[8] = {lo[0].x, lo[0].y, lo[0].z, lo[0].w, hi[0].x, hi[0].y, hi[0].z, hi[0].w};
#pragma unroll
        for (int s = 1; s < 8; ++s)
            if (s < S) {
                v[0] += lo[s].x; v[1] += lo[s].y; v[2] += lo[s].z; v[3] += lo[s].w;
                v[4] += hi[s].x; v[5] += hi[s].y; v[6] += hi[s].z; v[7] += hi[s].w;
            }
        if (colscale) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= load_scale<SK>(ws, (size_t)col + j);
        }
        float bv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (bias) {
#pragma unroll
            for (int j = 0; j < 8; ++j) bv[j] = bias[col + j];
        }
        const float xr = xs ? xs[row] : 1.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = xs ? fmaf(v[j], xr, bv[j]) : v[j] + bv[j];
        if constexpr (YDT == TFP8_F32) {
            *(float4*)((float*)y + i) = make_float4(v[0], v[1], v[2], v[3]);
            *(float4*)((float*)y + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
        } else {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t l = YDT == TFP8_BF16 ? f32_to_bf16_bits(v[2 * j]) : f32_to_f16_bits(v[2 * j]);
                const uint32_t h = YDT == TFP8_BF16 ? f32_to_bf16_bits(v[2 * j + 1]) : f32_to_f16_bits(v[2 * j + 1]);
                w[j] = l | (h << 16);
            }
            *(uint4*)((uint16_t*)y + i) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                                            const void* __restrict__ ws, int sk, int colscale,
                                                            const float* __restrict__ xs,
                                                            const float* __restrict__ bias, void* __restrict__ y,
                                                            int ydt) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int row = (int)(i / N), col = (int)(i % N);
        float v = part[i];
        for (int s = 1; s < S; ++s) v += part[(size_t)s * total + i];
        if (colscale) v *= scale_at(ws, sk, (size_t)col);
        const float bv = bias ? bias[col] : 0.f;
        store_elem(y, (size_t)i, ydt, xs ? fmaf(v, xs[row], bv) : v + bv);
    }
}

// ------------------------------------------------------------------ planning
struct GemmPlan {
    int bm, bn, wm, wn, bk;   // tile config
    int slices;               // split-K factor (1 = none)
};

static const GemmPlan GEMM_CFGS[] = {
    {0, 0, 0, 0, 0, 1},
    {16, 64, 1, 4, 64, 1},  {32, 64, 2, 2, 64, 1},   {64, 64, 2, 2, 64, 1},    {64, 128, 2, 2, 64, 1},
    {128, 128, 2, 2, 64, 1}, {128, 128, 4, 2, 64, 1}, {128, 128, 2, 4, 64, 1},  {256, 128, 4, 2, 64, 1},
    {128, 64, 4, 2, 64, 1}, {128, 128, 2, 4, 128, 1}, {128, 128, 4, 2, 128, 1}, {128, 256, 2, 4, 64, 1},
    {128, 256, 2, 4, 128, 1},
};
constexpr int GEMM_NCFG = (int)(sizeof(GEMM_CFGS) / sizeof(GEMM_CFGS[0]));

// Tile config by M (sweep on MI355X, K = N = 8192): above 128 rows the 128 x 256 tile with
// 128-wide K steps (8 waves, 2 per SIMD), or 128 x 128 with K-group scales, whose extra fp32
// partial accumulators would spill the larger tile.  Split K until the grid has a block per CU
// (two for the 4-wave tiles), keeping slices long next to the fp32 partials they produce.
GemmPlan gemm_plan(int M, int N, int K, bool grouped) {
    GemmPlan p;
    if (M <= 16) p = GEMM_CFGS[1];
    else if (M <= 32) p = GEMM_CFGS[2];
    else if (M <= 64) p = GEMM_CFGS[3];
    else if (M <= 128) p = GEMM_CFGS[4];
    else p = grouped ? GEMM_CFGS[7] : GEMM_CFGS[13];
    const int forced = tune(TUNE_GEMM_TILE);   // knob TFP8_GEMM_TILE: index into GEMM_CFGS
    if (forced > 0 && forced < GEMM_NCFG) p = GEMM_CFGS[forced];
    const long tiles = (long)((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
    const long want = p.wm * p.wn == 8 ? 256 : 512;
    int s = 1;
    while (tiles * s < want && s < 8 && (K / (s * 2)) >= 1024) s *= 2;
    const int fs = tune(TUNE_GEMM_SPLITK);
    if (fs > 0) s = std::min(fs, 8);
    p.slices = s;
    return p;
}

size_t gemm_stream_partial_bytes(int M, int N, int K, int G, int ws_kind);
size_t gemm_direct_partial_bytes(int M, int N, int K);

// Workspace for either GEMM kernel's split-K partials (the streaming kernel's split is sized
// with per-channel alignment, an upper bound for every group size).
size_t gemm_partial_bytes(int M, int N, int K) {
    const GemmPlan p = gemm_plan(M, N, K, false), q = gemm_plan(M, N, K, true);
    const int sl = std::max(p.slices, q.slices);
    const size_t v1 = sl > 1 ? (size_t)sl * M * N * sizeof(float) : 0;
    return std::max({v1, gemm_stream_partial_bytes(M, N, K, K, TFP8_SCALE_F32), gemm_direct_partial_bytes(M, N, K)});
}

// XCD column width of a GEMM grid whose blocks take tile ids (b & 7) * (nt / 8) + (b >> 3), walking
// ntm row tiles first (so XCD x owns whole column tiles [x * ntn / 8, (x + 1) * ntn / 8)), or 0.
int gemm_xcd_cols(int ntm, int ntn, int bn) {
    return ntn % 8 == 0 && ntm >= 1 ? ntn / 8 * bn : 0;
}

void splitk_reduce_launch(const float* part, int S, int M, int N, const void* ws, int sk, int colscale, const float* xs,
                          const float* bias, void* y, int ydt, int xcw, hipStream_t s) {
    if (N % 8 == 0 && S <= 8 && (uintptr_t)y % 16 == 0) {
        if (xcw % 8 || xcw >= N) xcw = 0;
        unsigned grid = grid_for((int64_t)M * N / 8, 256);
        if (xcw) grid = (grid + 7) / 8 * 8;
#define TFP8_RED(YD, SKV) \
    splitk_reduce8_kernel<YD, SKV><<<grid, 256, 0, s>>>(part, S, M, N, ws, colscale, xs, bias, y, xcw)
        if (sk == TFP8_SCALE_UE8M0) {
            if (ydt == TFP8_F32) TFP8_RED(TFP8_F32, TFP8_SCALE_UE8M0);
            else if (ydt == TFP8_BF16) TFP8_RED(TFP8_BF16, TFP8_SCALE_UE8M0);
            else TFP8_RED(TFP8_F16, TFP8_SCALE_UE8M0);
        } else {
            if (ydt == TFP8_F32) TFP8_RED(TFP8_F32, TFP8_SCALE_F32);
            else if (ydt == TFP8_BF16) TFP8_RED(TFP8_BF16, TFP8_SCALE_F32);
            else TFP8_RED(TFP8_F16, TFP8_SCALE_F32);
        }
#undef TFP8_RED
    } else {
        splitk_reduce_kernel<<<grid_for((int64_t)M * N, 256), 256, 0, s>>>(part, S, M, N, ws, sk, colscale, xs, bias, y,
                                                                          ydt);
    }
}

int run_gemm_stream(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
                    const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype,
                    float* partial, hipStream_t s);
int run_gemm_direct(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
                    const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype,
                    float* partial, hipStream_t s);
int run_gemv_mfma(const void* x, int x_dtype, const float* xs, int M, int K, const uint8_t* w, int N, const void* ws,
                  int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, hipStream_t s);
int gemv_mfma_min_m();

template <typename T, int FMT, int BM, int BN, int WM, int WN, int BK>
static void launch_gemm_cfg(const void* x, const float* xs, const uint8_t* w, const void* ws, int sk,
                            const float* bias, void* y, int ydt, int M, int N, int K, int G, int ng, float* part,
                            int slices, int slice_len, hipStream_t s) {
    const int nt = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    dim3 grid(nt, slices);
    if (ng > 1)
        gemm_kernel<T, FMT, BM, BN, WM, WN, BK, true><<<grid, 64 * WM * WN, 0, s>>>(
            (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, part, slice_len);
    else
        gemm_kernel<T, FMT, BM, BN, WM, WN, BK, false><<<grid, 64 * WM * WN, 0, s>>>(
            (const T*)x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, part, slice_len);
}

template <typename T, int FMT>
static void launch_gemm_t(const GemmPlan& p, const void* x, const float* xs, const uint8_t* w, const void* ws,
                          int sk, const float* bias, void* y, int ydt, int M, int N, int K, int G, int ng,
                          float* part, int slices, int slice_len, hipStream_t s) {
#define TFP8_GEMM_CFG(BM_, BN_, WM_, WN_, BK_)                                                               \
    if (p.bm == BM_ && p.bn == BN_ && p.wm == WM_ && p.wn == WN_ && p.bk == BK_) {                            \
        launch_gemm_cfg<T, FMT, BM_, BN_, WM_, WN_, BK_>(x, xs, w, ws, sk, bias, y, ydt, M, N, K, G, ng, part, \
                                                         slices, slice_len, s);                              \
        return;                                                                                             \
    }
    TFP8_GEMM_CFG(16, 64, 1, 4, 64)
    TFP8_GEMM_CFG(32, 64, 2, 2, 64)
    TFP8_GEMM_CFG(64, 64, 2, 2, 64)
    TFP8_GEMM_CFG(64, 128, 2, 2, 64)
    TFP8_GEMM_CFG(128, 128, 2, 2, 64)
    TFP8_GEMM_CFG(128, 128, 4, 2, 64)
    TFP8_GEMM_CFG(128, 128, 2, 4, 64)
    TFP8_GEMM_CFG(256, 128, 4, 2, 64)
    TFP8_GEMM_CFG(128, 64, 4, 2, 64)
    TFP8_GEMM_CFG(128, 128, 2, 4, 128)
    TFP8_GEMM_CFG(128, 128, 4, 2, 128)
    TFP8_GEMM_CFG(128, 256, 2, 4, 64)
    TFP8_GEMM_CFG(128, 256, 2, 4, 128)
#undef TFP8_GEMM_CFG
}

static int gcd_i(int a, int b) { while (b) { int t = a % b; a = b; b = t; } return a; }

// Validated by the caller.  x16 is f16 or bf16 [M,K]; xs optional.  partial: workspace of
// gemm_partial_bytes() (may be null when that is 0).
int run_gemm(const void* x16, int x16_dtype, const float* xs, int M, int K, const uint8_t* w, int N,
             const void* ws, int ws_kind, int G, int fmt, const float* bias, void* y, int y_dtype, float* partial,
             hipStream_t s) {
    // Up to 16 rows go to the matrix-core decode kernel (no split-K; on MI355X it beats the
    // weight-streaming kernel at every M from 9 to 16: C3 M=16 15.7 vs 16.9 us, C2 M=16 16.7 vs
    // 20.7 us); then the direct-to-LDS GEMM (one scale per weight row, from its minimum M up), the
    // weight-streaming kernel (M <= 128) and the LDS-tiled kernel below, the general path.
    if (M <= tune(TUNE_GEMV_MFMA_MAX_M) && M >= gemv_mfma_min_m()) {
        const int rm = run_gemv_mfma(x16, x16_dtype, xs, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, s);
        if (rm != NOT_TAKEN) return rm;
    }
    const int rd = run_gemm_direct(x16, x16_dtype, xs, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, partial, s);
    if (rd != NOT_TAKEN) return rd;
    const int rs = run_gemm_stream(x16, x16_dtype, xs, M, K, w, N, ws, ws_kind, G, fmt, bias, y, y_dtype, partial, s);
    if (rs != NOT_TAKEN) return rs;
    const int ng = K / G;
    GemmPlan p = gemm_plan(M, N, K, ng > 1);
    int slices = p.slices, slice_len = K;
    if (slices > 1) {
        // Slices are whole K tiles, and whole K groups when the scales are grouped.
        int align = p.bk;
        if (ng > 1) align = p.bk / gcd_i(p.bk, G) * G;
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
    const int xcw = (((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn)) % 8 == 0
                        ? gemm_xcd_cols((M + p.bm - 1) / p.bm, (N + p.bn - 1) / p.bn, p.bn) : 0;
    splitk_reduce_launch(part, slices, M, N, ws, ws_kind, ng == 1 ? 1 : 0, xs, bias, y, y_dtype, xcw, s);
    return check_launch("tfp8_gemm splitk reduce");
}

}  // namespace tfp8
