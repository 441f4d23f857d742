// Streaming FP8-weight GEMV for M <= 8 rows (the decode step): kernel and launch configurations.
//
// y[m,n] = sum_c s(n, c) * sum_{t<16} x[m, c+t] * decode(w[n, c+t]) + bias[n]   (c = 16-chunks)
// which is the formula of the reference GEMV (tfp8/csrc/tfp8_kernels.cu:171-269), laid out for
// CDNA4 instead of 32-lane warps:
//   * a wave owns R weight rows at a time and reads each 1 KB per instruction: one
//     buffer_load_dwordx4 per lane through a buffer resource covering the R rows (SGPRs), with the
//     row and chunk offsets in the scalar offset and a fixed 16*lane vector offset;
//   * a block owns a contiguous run of row groups and its waves take them round-robin; a wave's
//     work is the list of (row group, 1 KB chunk) items, and the loads of the next 2U items are
//     always in flight while U items are decoded and accumulated -- the prefetch runs across row
//     boundaries, so a wave never drains its loads between rows;
//   * every load is unconditional: items past the end use an empty buffer resource, lanes past K
//     in a partial last chunk use an out-of-range offset, and rows past N fall outside the
//     group's resource -- the hardware returns zeros for all of them, so the main loop has no
//     branches around memory and the compiler can wait for exactly the load it needs;
//   * the activation rows (M x K, native dtype) and the K-group scales of the block's rows (as
//     f32) are copied once per block into LDS; when a row group is finished the wave reduces it
//     and writes its R adjacent outputs per activation row (with per-channel scale and bias) in
//     one packed store -- at the end of a GEMV the output stores are on the critical path;
//   * codes are decoded in registers with v_cvt_scalef32_pk_{bf16,f16}_{fp8,bf8} (2 codes per
//     instruction), no LDS table; 16-bit activations are multiplied with v_dot2_f32_{bf16,f16}
//     (exact products, fp32 accumulation); fp32 activations use v_cvt_pk_f32_fp8 and fp32 FMA;
//   * a row group is reduced with 4 DPP adds per 16-lane row (quad_perm x2, row_half_mirror,
//     row_mirror) and 4 v_readlane.
#pragma once
#include <algorithm>
#include <atomic>

#include "tfp8_common.h"

namespace tfp8 {

constexpr int GEMV_SLDS_MAX = 16 * 1024;     // K-group scale bytes staged in LDS per block
constexpr int GEMV_CHUNK = 1024;             // bytes of one row read by one wave instruction
constexpr int GEMV_MAX_ROWS_PER_BLOCK = 1024;
constexpr uint32_t BUF_FLAGS = 0x00020000u;  // buffer resource word 3 for gfx9 (raw, 32-bit format)
constexpr uint32_t BUF_OOB = 0x80000000u;    // an offset beyond every resource used here
constexpr int BUF_NT = 2;                    // cache policy: non-temporal (streamed once)

__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float c, int xdt) {
    if (xdt == TFP8_BF16)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// Sum over the 64 lanes of a wave; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, (int)BUF_FLAGS);
}
template <int AUX = 0>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX));
}

// R consecutive outputs y[o .. o+R) of runtime dtype: one 2R- or 4R-byte store when `pack`
// (o % R == 0 and y aligned), else one element at a time; only the first nval are written.
template <int R>
__device__ __forceinline__ void store_rows(void* y, size_t o, int ydt, const float (&v)[R], int nval, bool pack) {
    if (pack && nval == R) {
        if (ydt == TFP8_F32) {
            if constexpr (R == 2) { *(float2*)((float*)y + o) = make_float2(v[0], v[1]); return; }
            if constexpr (R == 4) { *(float4*)((float*)y + o) = make_float4(v[0], v[1], v[2], v[3]); return; }
        } else {
            uint32_t h[R];
#pragma unroll
            for (int r = 0; r < R; ++r) h[r] = ydt == TFP8_BF16 ? f32_to_bf16_bits(v[r]) : f32_to_f16_bits(v[r]);
            if constexpr (R == 2) { *(uint32_t*)((uint16_t*)y + o) = h[0] | (h[1] << 16); return; }
            if constexpr (R == 4) {
                *(uint2*)((uint16_t*)y + o) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                return;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < nval) store_elem(y, o + r, ydt, v[r]);
}

template <int MT, int XDT, int FMT, bool GROUPED, int R, int U, int TPB, bool XLDS>
__global__ __launch_bounds__(TPB) void gemv_kernel(
    const void* __restrict__ x, const uint8_t* __restrict__ w, const void* __restrict__ ws, int sk,
    const float* __restrict__ bias, void* __restrict__ y, int ydt, int M, int N, int K, int G, int ng,
    int gshift, int per_block, int xlds_bytes, int slds_bytes, int ldy) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int XB = XDT == TFP8_F32 ? 4 : 2;
    constexpr int GEMV_THREADS = TPB, GEMV_WAVES = TPB / 64;
    const int tid = threadIdx.x, lane = tid & 63;
    // The wave index is wave-uniform; readfirstlane makes every cursor and row base below scalar.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ngr = (N + R - 1) / R;                         // row groups
    // Blocks are dispatched round-robin over the 8 XCDs; renumber them so that each XCD owns one
    // contiguous run of rows (a bijection for any grid size).  Each 128-byte line of y is then
    // written from a single XCD's L2 instead of partially from all eight.
    const int nblk = gridDim.x, xcd = blockIdx.x & 7, q8 = nblk >> 3, r8 = nblk & 7;
    const int lb = xcd * q8 + min(xcd, r8) + (blockIdx.x >> 3);
    const int gb = lb * per_block;                           // first row group of this block
    const int ge = min(ngr, gb + per_block);
    const int nmine = ge - gb > wave ? (ge - gb - wave + GEMV_WAVES - 1) / GEMV_WAVES : 0;
    const int cpr = (K + GEMV_CHUNK - 1) / GEMV_CHUNK;       // chunks per row
    const int items = nmine * cpr;
    const int row0 = gb * R;                                 // first row of this block
    const int rows_b = min(N, ge * R) - row0;                // rows of this block
    float* ssc = (float*)(smem + xlds_bytes);                // block scales, f32 [rows][ng] or [rows]

    const uint32_t lane16 = (uint32_t)lane * 16u;
    // Vector offset of the last chunk of a row: lanes past K read out of range (zeros).
    const uint32_t last_off = (uint32_t)((cpr - 1) * GEMV_CHUNK) + lane16;
    const uint32_t voff_last = last_off < (uint32_t)K ? lane16 : BUF_OOB;
    const int kx_last = min((int)last_off, K - 16);          // clamped activation index there

    // ---------------------------------------------------------------- load side
    // One buffer resource spans the whole weight matrix (the host keeps N*K < 2^31); a load's
    // scalar offset is row*K + chunk*1024. Rows past N and items past the end use offset N*K,
    // i.e. out of range, and read zeros.
    const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(w, (uint32_t)N * (uint32_t)K);
    const uint32_t oob = (uint32_t)N * (uint32_t)K;
    int lt = 0, lc = 0;   // (row group ordinal, chunk) of the next item to load
    auto issue = [&](uint4 (&buf)[U][R]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int n0 = (gb + wave + GEMV_WAVES * lt) * R;
            const uint32_t base = (uint32_t)n0 * (uint32_t)K + (uint32_t)(lc * GEMV_CHUNK);
            const uint32_t voff = lc == cpr - 1 ? voff_last : lane16;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const bool ok = lt < nmine && n0 + r < N;
                buf[u][r] = buf_load16<BUF_NT>(wrs, voff, ok ? base + (uint32_t)(r * K) : oob);
            }
            if (++lc == cpr) { lc = 0; ++lt; }
        }
    };

    uint4 sa[U][R], sb[U][R];

    // Block-constant data staged in LDS: activations, then the scales (K-group scales of the block's
    // rows, or their per-channel scale), then the bias. The first slice of each copy is loaded
    // before the weight prefetch is issued and written after it, so the waits it needs never
    // cover a weight load.
    const int srows = max(rows_b, 0);
    const int scount = GROUPED ? srows * ng : srows;         // f32 scale values staged
    float* sbias = (float*)(smem + xlds_bytes + slds_bytes); // [rows]
    // R adjacent outputs go out as one store when y and every row's offset allow it.
    const bool ypack = R > 1 && (reinterpret_cast<uintptr_t>(y) % (R * (ydt == TFP8_F32 ? 4 : 2))) == 0 && ldy % R == 0;
    const bool ue8 = sk == TFP8_SCALE_UE8M0;
    const size_t s0 = GROUPED ? (size_t)row0 * ng : (size_t)row0;
    const __amdgpu_buffer_rsrc_t srs = buf_rsrc(ws, (uint32_t)((size_t)N * ng * (ue8 ? 1 : 4)));
    const __amdgpu_buffer_rsrc_t brs = buf_rsrc(bias, bias ? (uint32_t)(N * 4) : 0u);
    auto scale_raw = [&](int i) -> uint32_t {
        return ue8 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(srs, (int)(s0 + i), 0, 0)
                   : __builtin_amdgcn_raw_buffer_load_b32(srs, (int)((s0 + i) * 4), 0, 0);
    };
    auto scale_f32 = [&](uint32_t raw) { return ue8 ? ue8m0_to_f32(raw) : __uint_as_float(raw); };

    constexpr int XC = 2;
    uint4 xcp[XC];
    const int x16n = xlds_bytes >> 4;
    if constexpr (XLDS) {
        const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, (uint32_t)xlds_bytes);
#pragma unroll
        for (int q = 0; q < XC; ++q) xcp[q] = buf_load16(xr, (uint32_t)(tid + q * GEMV_THREADS) * 16u, 0);
    }
    const uint32_t scp = tid < scount ? scale_raw(tid) : 0u;
    // (no bias: no load -- every load instruction here costs address-unit time the weights need)
    const uint32_t bcp = bias ? __builtin_amdgcn_raw_buffer_load_b32(brs, (row0 + tid) * 4, 0, 0) : 0u;

    issue(sa);
    issue(sb);

    if constexpr (XLDS) {
#pragma unroll
        for (int q = 0; q < XC; ++q)
            if (tid + q * GEMV_THREADS < x16n) ((uint4*)smem)[tid + q * GEMV_THREADS] = xcp[q];
        for (int i = tid + XC * GEMV_THREADS; i < x16n; i += GEMV_THREADS) ((uint4*)smem)[i] = ((const uint4*)x)[i];
    }
    if (tid < scount) ssc[tid] = scale_f32(scp);
    for (int i = tid + GEMV_THREADS; i < scount; i += GEMV_THREADS) ssc[i] = scale_f32(scale_raw(i));
    if (tid < srows) sbias[tid] = __uint_as_float(bcp);
    if (bias)
        for (int i = tid + GEMV_THREADS; i < srows; i += GEMV_THREADS)
            sbias[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(brs, (row0 + i) * 4, 0, 0));
    else
        for (int i = tid + GEMV_THREADS; i < srows; i += GEMV_THREADS) sbias[i] = 0.f;
    __syncthreads();

    // ---------------------------------------------------------------- compute side
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

    auto xrow = [&](int m, int kk) -> const uint4* {
        const int off = (m * K + kk) * XB;
        if constexpr (XLDS) return (const uint4*)(smem + off);
        else return (const uint4*)((const uint8_t*)x + off);
    };

    int ct = 0, cc = 0;   // (row group ordinal, chunk) of the next item to compute
    auto compute = [&](const uint4 (&buf)[U][R], int i0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (i0 + u < items) {
                const bool last = cc == cpr - 1;
                const int kk = last ? kx_last : cc * GEMV_CHUNK + (int)lane16;
                const bool valid = !last || voff_last != BUF_OOB;
                const int rl = (wave + GEMV_WAVES * ct) * R;     // row of slot 0, relative to row0
                float sc[R];
                if constexpr (GROUPED) {
                    const int g = gshift >= 0 ? (kk >> gshift) : kk / G;
#pragma unroll
                    for (int r = 0; r < R; ++r) sc[r] = ssc[min(rl + r, rows_b - 1) * ng + g];
                }
                float part[R][MT];
                if constexpr (XDT == TFP8_F32) {
                    float wf[R][16];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        dec4_f32<FMT>(buf[u][r].x, wf[r]);
                        dec4_f32<FMT>(buf[u][r].y, wf[r] + 4);
                        dec4_f32<FMT>(buf[u][r].z, wf[r] + 8);
                        dec4_f32<FMT>(buf[u][r].w, wf[r] + 12);
                    }
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m < M) {
                            const uint4* xp = xrow(m, kk);
                            float xf[16];
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const uint4 v = xp[q];
                                xf[4 * q] = __uint_as_float(v.x); xf[4 * q + 1] = __uint_as_float(v.y);
                                xf[4 * q + 2] = __uint_as_float(v.z); xf[4 * q + 3] = __uint_as_float(v.w);
                            }
#pragma unroll
                            for (int r = 0; r < R; ++r) {
                                float a = 0.f;
#pragma unroll
                                for (int q = 0; q < 16; ++q) a = fmaf(xf[q], wf[r][q], a);
                                part[r][m] = a;
                            }
                        }
                    }
                } else {
                    uint32_t wk[R][8];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t d[4] = {buf[u][r].x, buf[u][r].y, buf[u][r].z, buf[u][r].w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            wk[r][2 * q] = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[q], false) : cvt2_f16<FMT>(d[q], false);
                            wk[r][2 * q + 1] = XDT == TFP8_BF16 ? cvt2_bf16<FMT>(d[q], true) : cvt2_f16<FMT>(d[q], true);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m < M) {
                            const uint4* xp = xrow(m, kk);
                            const uint4 v0 = xp[0], v1 = xp[1];
                            const uint32_t xv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                            for (int r = 0; r < R; ++r) {
                                float a = 0.f;
#pragma unroll
                                for (int q = 0; q < 8; ++q) a = dot2_acc(xv[q], wk[r][q], a, XDT);
                                part[r][m] = a;
                            }
                        }
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m < M) {
                            const float p = valid ? part[r][m] : 0.f;
                            acc[r][m] = GROUPED ? fmaf(p, sc[r], acc[r][m]) : acc[r][m] + p;
                        }
                    }
                if (last) {
                    // Row group finished: lane m takes the R row totals of activation row m and
                    // writes them straight to y, R adjacent outputs in one store when aligned.
                    float v[R];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float t = 0.f;
#pragma unroll
                        for (int m = 0; m < MT; ++m) {
                            const float tot = wave_sum(acc[r][m]);
                            t = lane == m ? tot : t;
                            acc[r][m] = 0.f;
                        }
                        v[r] = t;
                    }
                    if (lane < M) {
                        const int nval = min(R, rows_b - rl);
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const int rr = min(rl + r, rows_b - 1);
                            v[r] = v[r] * (GROUPED ? 1.f : ssc[rr]) + sbias[rr];
                        }
                        store_rows<R>(y, (size_t)lane * ldy + row0 + rl, ydt, v, nval, ypack);
                    }
                }
                if (++cc == cpr) { cc = 0; ++ct; }
            }
        }
    };

    // Stages past the last item are not issued (a uniform branch): out-of-range loads return
    // zeros without touching memory but still occupy the address units.
    for (int i0 = 0; i0 < items; i0 += 2 * U) {
        compute(sa, i0);
        if (i0 + 2 * U < items) issue(sa);
        compute(sb, i0 + U);
        if (i0 + 3 * U < items) issue(sb);
    }

}

// Compiled configurations (id, R, U, waves per CU, threads per block); gemv_pick() chooses one
// by shape and the knob TFP8_GEMV_CFG=<id> overrides it.
#ifdef TFP8_GEMV_SWEEP
#define TFP8_GEMV_CFG_LIST X(0, 1, 2, 32, 256) X(1, 1, 2, 64, 256) X(2, 1, 2, 64, 512) X(3, 1, 2, 64, 1024) \
    X(4, 2, 2, 32, 256) X(5, 2, 2, 32, 1024) X(6, 1, 4, 32, 1024) X(7, 4, 2, 16, 256) X(8, 2, 4, 16, 512) \
    X(9, 2, 1, 32, 256) X(10, 2, 4, 32, 256) X(11, 2, 2, 32, 512) X(12, 1, 4, 32, 256) X(13, 4, 1, 32, 256) \
    X(14, 1, 1, 32, 256) X(15, 2, 2, 32, 128) X(16, 1, 2, 32, 128) X(17, 2, 2, 28, 448) X(18, 1, 2, 56, 448)
#else
#define TFP8_GEMV_CFG_LIST X(2, 1, 2, 64, 512) X(4, 2, 2, 32, 256) X(8, 2, 4, 16, 512) X(17, 2, 2, 28, 448)
#endif

// Per-device attributes, queried once: CU count and the LDS bytes one block may use.  Callers on
// several host threads may fill an entry at the same time (with the same values): the LDS size is
// stored before the CU count is published (release), and a reader that sees the CU count
// (acquire) sees the LDS size.
struct DevInfo { int cus, lds; };
static inline DevInfo dev_info() {
    static std::atomic<int> cus[64], lds[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return {256, 64 * 1024};
    int c = cus[dev].load(std::memory_order_acquire);
    if (!c) {
        int v = 0, l = 0;
        const bool ok = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0;
        const bool okl = hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && l > 0;
        lds[dev].store(okl ? l : 64 * 1024, std::memory_order_relaxed);
        c = ok ? v : 256;
        cus[dev].store(c, std::memory_order_release);
    }
    return {c, lds[dev].load(std::memory_order_relaxed)};
}

// Config by shape; sized from a sweep on MI355X.  Every config is correct for every shape.
static inline int gemv_pick(int M, int N) {
    const int forced = tune(TUNE_GEMV_CFG);
    if (forced >= 0) return forced;
    (void)N;
    if (M <= 1) return 4;
    if (M <= 4) return 2;
    return 8;
}

template <int MT, int XDT, int FMT, bool GROUPED, int R, int U, int TPB>
static void launch_rows(int waves_per_cu, const void* x, const uint8_t* w, const void* ws, int sk, const float* bias,
                        void* y, int ydt, int M, int N, int K, int G, int ng, int gshift, int ldy, hipStream_t s) {
    const int ngr = (N + R - 1) / R;
    const int wpc = tune(TUNE_GEMV_WPC) > 0 ? tune(TUNE_GEMV_WPC) : waves_per_cu;
    const DevInfo di = dev_info();
    long waves = (long)di.cus * wpc;
    if (waves > ngr) waves = ngr;
    constexpr int GEMV_WAVES = TPB / 64;
    int grid = (int)((waves + GEMV_WAVES - 1) / GEMV_WAVES);
    int per_block = (ngr + grid - 1) / grid;
    // Bound the block's rows (LDS for results, and for K-group scales when grouped).
    long max_groups = GEMV_MAX_ROWS_PER_BLOCK / R;
    if (GROUPED) max_groups = std::min<long>(max_groups, GEMV_SLDS_MAX / (4L * ng * R));
    if (max_groups < 1) max_groups = 1;
    if (per_block > max_groups) per_block = (int)max_groups;
    grid = (ngr + per_block - 1) / per_block;
    const size_t xbytes = (size_t)M * K * (XDT == TFP8_F32 ? 4 : 2);
    const size_t sbytes = ((size_t)per_block * R * (GROUPED ? ng : 1) * 4 + 15) / 16 * 16;
    const size_t obytes = (size_t)per_block * R * 4;   // bias
    const bool xlds = xbytes + sbytes + obytes <= (size_t)di.lds;
    const int xl = xlds ? (int)xbytes : 0;
    if (xlds)
        gemv_kernel<MT, XDT, FMT, GROUPED, R, U, TPB, true><<<grid, TPB, xl + sbytes + obytes, s>>>(
            x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, per_block, xl, (int)sbytes, ldy);
    else
        gemv_kernel<MT, XDT, FMT, GROUPED, R, U, TPB, false><<<grid, TPB, sbytes + obytes, s>>>(
            x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, per_block, 0, (int)sbytes, ldy);
}

// Weight offsets inside a launch are 32-bit: a matrix of 2^31 bytes or more is run as several
// launches over row ranges (output columns), each below that size.
template <int MT, int XDT, int FMT, bool GROUPED, int R, int U, int TPB>
static void launch_cfg(int waves_per_cu, const void* x, const uint8_t* w, const void* ws, int sk, const float* bias,
                       void* y, int ydt, int M, int N, int K, int G, int ng, int gshift, hipStream_t s) {
    const long max_rows = std::max<long>(1, ((1L << 31) - 1) / K / R * R);
    const int ysz = ydt == TFP8_F32 ? 4 : 2;
    const int ssz = sk == TFP8_SCALE_UE8M0 ? 1 : 4;
    for (long n0 = 0; n0 < N; n0 += max_rows) {
        const int nr = (int)std::min<long>(max_rows, N - n0);
        launch_rows<MT, XDT, FMT, GROUPED, R, U, TPB>(waves_per_cu, x, w + n0 * K, (const uint8_t*)ws + n0 * ng * ssz, sk,
                                                      bias ? bias + n0 : nullptr, (uint8_t*)y + n0 * ysz, ydt, M, nr,
                                                      K, G, ng, gshift, N, s);
    }
}

template <int MT, int XDT, int FMT, bool GROUPED>
static void launch_m(const void* x, const uint8_t* w, const void* ws, int sk, const float* bias, void* y, int ydt,
                     int M, int N, int K, int G, int ng, int gshift, hipStream_t s) {
    const int c = gemv_pick(M, N);
#define X(ID, R_, U_, WPC_, TPB_)                                                                              \
    if (c == ID) {                                                                                             \
        launch_cfg<MT, XDT, FMT, GROUPED, R_, U_, TPB_>(WPC_, x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, \
                                                        s);                                                    \
        return;                                                                                                \
    }
    TFP8_GEMV_CFG_LIST
#undef X
    launch_cfg<MT, XDT, FMT, GROUPED, 2, 2, 256>(32, x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);  // unknown id
}

template <int XDT, int FMT, bool GROUPED>
static void launch_gemv_m(const void* x, const uint8_t* w, const void* ws, int sk, const float* bias, void* y,
                          int ydt, int M, int N, int K, int G, int ng, int gshift, hipStream_t s) {
    if (M <= 1) launch_m<1, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
    else if (M <= 2) launch_m<2, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
    else if (M <= 4) launch_m<4, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
    else launch_m<8, XDT, FMT, GROUPED>(x, w, ws, sk, bias, y, ydt, M, N, K, G, ng, gshift, s);
}

}  // namespace tfp8
