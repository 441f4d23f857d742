// Fused ops of one decoding position of the example Llama model (tfp8/examples/demo_llm.py), the
// work between its FP8 linears: each op is one kernel where the PyTorch form of the same step runs
// a chain of elementwise kernels (about 60 launches per layer become 6).  Every op keeps that
// form's roundings -- bf16 results rounded where it rounds them, fp32 arithmetic in its order,
// no contracted multiply-adds -- so the two forms differ only in the order of the fp32 sums
// (the RMS of a row, the attention dot products and softmax sums).
//
// Built as libtfp8_llm.so beside the example (C ABI: device pointers, sizes, a hipStream_t passed
// as void*); it is the example model's own code, not part of the FP8 library's interface.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

// Every multiply, add and subtract below is rounded on its own, as PyTorch's separate kernels
// round them: hipcc contracts a * b + c into v_fma_f32 by default (so do HIP's __fmul_rn and
// __fadd_rn, which are the plain operators), and x1 c - x2 s as fma(x1, c, -x2 s) changes a bf16
// result now and then.  The multiply-adds that may fuse are written as fmaf.
#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ float mul_rn(float a, float b) { return a * b; }
__device__ __forceinline__ float add_rn(float a, float b) { return a + b; }
__device__ __forceinline__ float sub_rn(float a, float b) { return a - b; }

__device__ __forceinline__ float bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even (torch's conversion); NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t to_bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = add_rn(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
// Sum / max over a 256-thread block (every thread gets the result); red holds 4 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return add_rn(add_rn(red[0], red[1]), add_rn(red[2], red[3]));
}
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// h = x + r (bf16 add; r null: h = x) and y = bf16((float(h) * rsqrt(mean(float(h)^2) + eps)) * float(w)),
// the RMSNorm of demo_llm.RMSNorm.forward.  One 256-thread block per row, CH chunks of 8 elements
// per thread (d % 8 == 0, d <= 2048 CH).
template <int CH>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ r,
                                                          uint16_t* __restrict__ h, uint16_t* __restrict__ y,
                                                          const uint16_t* __restrict__ w, int d, float eps) {
    __shared__ float red[4];
    const size_t base = (size_t)blockIdx.x * d;
    float v[CH][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = (c * 256 + (int)threadIdx.x) * 8;
        if (i < d) {
            const uint4 xa = *(const uint4*)(x + base + i);
            const uint16_t* xs = (const uint16_t*)&xa;
            uint4 ha = xa;
            uint16_t* hs = (uint16_t*)&ha;
            if (r) {
                const uint4 ra = *(const uint4*)(r + base + i);
                const uint16_t* rs = (const uint16_t*)&ra;
#pragma unroll
                for (int j = 0; j < 8; ++j) hs[j] = to_bf(add_rn(bf(xs[j]), bf(rs[j])));
                *(uint4*)(h + base + i) = ha;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[c][j] = bf(hs[j]);
                ss = add_rn(ss, mul_rn(v[c][j], v[c][j]));
            }
        }
    }
    const float ms = __fdiv_rn(block_sum(ss, red), (float)d);
    const float inv = rsqrtf(add_rn(ms, eps));
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = (c * 256 + (int)threadIdx.x) * 8;
        if (i < d) {
            const uint4 wa = *(const uint4*)(w + i);
            const uint16_t* ws = (const uint16_t*)&wa;
            uint4 ya;
            uint16_t* ys = (uint16_t*)&ya;
#pragma unroll
            for (int j = 0; j < 8; ++j) ys[j] = to_bf(mul_rn(mul_rn(v[c][j], inv), bf(ws[j])));
            *(uint4*)(y + base + i) = ya;
        }
    }
}

// Rotary embedding of one position and the KV-cache write (demo_llm._rotary and the index_copy_ of
// Attention.forward_static): x = [x1, x2] -> bf16([x1 c - x2 s, x2 c + x1 s]).  Block (head, b),
// hd / 2 threads: heads below H are query heads (out: qf [B, H, hd] fp32, the rotated bf16 values
// widened); the next Hkv are key heads, written into the bf16 cache kt [B, Hkv, hd, L] at column
// *pos, with the value head into vc [B, Hkv, L, hd] at row *pos.  Row b of q / k / v starts ldq / ldk /
// ldv elements after row b - 1 (slices of one fused projection).  A position outside the cache
// writes nothing (the host checks it; this only keeps a bad position from writing out of bounds).
__global__ void rope_cache_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                  const uint16_t* __restrict__ v, const float* __restrict__ cs,
                                  const float* __restrict__ sn, float* __restrict__ qf, uint16_t* __restrict__ kt,
                                  uint16_t* __restrict__ vc, const int64_t* __restrict__ pos, int H, int Hkv, int hd,
                                  int L, int ldq, int ldk, int ldv) {
    const int head = blockIdx.x, b = blockIdx.y, i = threadIdx.x, half = hd / 2;
    const float c = cs[i], s = sn[i];
    if (head < H) {
        const uint16_t* src = q + (size_t)b * ldq + (size_t)head * hd;
        const float x1 = bf(src[i]), x2 = bf(src[i + half]);
        float* dst = qf + ((size_t)b * H + head) * hd;
        dst[i] = bf(to_bf(sub_rn(mul_rn(x1, c), mul_rn(x2, s))));
        dst[i + half] = bf(to_bf(add_rn(mul_rn(x2, c), mul_rn(x1, s))));
        return;
    }
    const int64_t p = *pos;
    if (p < 0 || p >= L) return;
    const int kh = head - H;
    const size_t hb = (size_t)b * Hkv + kh;
    const uint16_t* src = k + (size_t)b * ldk + (size_t)kh * hd;
    const float x1 = bf(src[i]), x2 = bf(src[i + half]);
    kt[(hb * hd + i) * L + p] = to_bf(sub_rn(mul_rn(x1, c), mul_rn(x2, s)));
    kt[(hb * hd + i + half) * L + p] = to_bf(add_rn(mul_rn(x2, c), mul_rn(x1, s)));
    const uint16_t* vs = v + (size_t)b * ldv + (size_t)kh * hd;
    vc[(hb * L + p) * hd + i] = vs[i];
    vc[(hb * L + p) * hd + i + half] = vs[i + half];
}

// The prefill's rotary embedding and cache write (Attention.forward: _rotary of q and k, then the
// cache slices at start .. start + T - 1).  Block (head, b * nt + tile): RP_T positions of one head,
// 256 threads, cos / sin fp32 [T, hd / 2].  Query heads write the rotated bf16 q into qo [B, H, T, hd]
// (the layout of the score product's left operand).  Key heads stage their rotated tile in LDS as
// [hd][RP_T] and write every row of kt [B, Hkv, hd, L] as RP_T contiguous positions (a position per
// thread would scatter 2-byte stores L elements apart); the value head goes straight to vc [B, Hkv,
// L, hd] rows.  The same operations as rope_cache_kernel, so the same bits as the PyTorch form.
constexpr int RP_T = 64;
template <int V>   // V consecutive dims per thread (V = 4: 8-byte q / k / v and 16-byte cos / sin accesses)
__global__ __launch_bounds__(256) void rope_prefill_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                           const uint16_t* __restrict__ v, const float* __restrict__ cs,
                                                           const float* __restrict__ sn, uint16_t* __restrict__ qo,
                                                           uint16_t* __restrict__ kt, uint16_t* __restrict__ vc, int start,
                                                           int T, int H, int Hkv, int hd, int L, int ldq, int ldk, int ldv) {
    extern __shared__ uint16_t tile[];                        // [hd][RP_T + 2]
    const int nt = (T + RP_T - 1) / RP_T, head = blockIdx.x, b = blockIdx.y / nt;
    const int t0 = (blockIdx.y - b * nt) * RP_T, cnt = min(RP_T, T - t0), half = hd / 2, hv = half / V;
    const bool is_q = head < H;
    const int kh = head - H;
    const size_t hb = (size_t)b * Hkv + kh;
    const int n = cnt * hv;
    typedef uint16_t u16v __attribute__((ext_vector_type(V)));
    typedef float f32v __attribute__((ext_vector_type(V)));
    for (int e0 = threadIdx.x; e0 < n; e0 += 4 * blockDim.x) {   // four loads of each kind in flight
        f32v c[4], sv[4];
        u16v x1[4], x2[4], v1[4], v2[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            if (e >= n) break;
            const int tl = e / hv, i = (e - tl * hv) * V, t = t0 + tl;
            const size_t bt = (size_t)b * T + t;
            c[u] = *(const f32v*)(cs + (size_t)t * half + i);
            sv[u] = *(const f32v*)(sn + (size_t)t * half + i);
            const uint16_t* src = is_q ? q + bt * ldq + (size_t)head * hd : k + bt * ldk + (size_t)kh * hd;
            x1[u] = *(const u16v*)(src + i);
            x2[u] = *(const u16v*)(src + i + half);
            if (!is_q) {
                const uint16_t* vs = v + bt * ldv + (size_t)kh * hd;
                v1[u] = *(const u16v*)(vs + i);
                v2[u] = *(const u16v*)(vs + i + half);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            if (e >= n) break;
            const int tl = e / hv, i = (e - tl * hv) * V, t = t0 + tl;
            u16v r1, r2;
#pragma unroll
            for (int w = 0; w < V; ++w) {
                const float a = bf(x1[u][w]), bb = bf(x2[u][w]);
                r1[w] = to_bf(sub_rn(mul_rn(a, c[u][w]), mul_rn(bb, sv[u][w])));
                r2[w] = to_bf(add_rn(mul_rn(bb, c[u][w]), mul_rn(a, sv[u][w])));
            }
            if (is_q) {
                uint16_t* dst = qo + (((size_t)b * H + head) * T + t) * hd;
                *(u16v*)(dst + i) = r1;
                *(u16v*)(dst + i + half) = r2;
            } else {
#pragma unroll
                for (int w = 0; w < V; ++w) {
                    tile[(i + w) * (RP_T + 2) + tl] = r1[w];
                    tile[(i + w + half) * (RP_T + 2) + tl] = r2[w];
                }
                uint16_t* vd = vc + (hb * L + start + t) * hd;
                *(u16v*)(vd + i) = v1[u];
                *(u16v*)(vd + i + half) = v2[u];
            }
        }
    }
    if (is_q) return;                                         // uniform over the block
    __syncthreads();
    const int tl = threadIdx.x % RP_T;
    for (int d = threadIdx.x / RP_T; d < hd; d += blockDim.x / RP_T)
        if (tl < cnt) kt[(hb * hd + d) * L + start + t0 + tl] = tile[d * (RP_T + 2) + tl];
}

// Decode attention over cache positions 0..*pos, split over gridDim.y chunks of at most 64
// positions of the bf16 caches (widened as read).  Block (b * H + h, j), 4 waves: lane l takes
// position t0 + l, wave w the dot product
// over head dimensions [w HD/4, (w+1) HD/4) (every load of a lane in flight at once), summed over
// the waves in LDS: s_t = (q . k_t) / sdiv.  Then m = max s_t, l = sum exp(s_t - m) and
// o[i] = sum exp(s_t - m) v_t[i], stored as part[(bh * S + j) * (HD + 2) + {0: m, 1: l, 2 + i: o[i]}]
// (an empty chunk stores m = -inf, l = 0, o = 0).  Query head h reads key/value head h / (H / Hkv)
// (repeat_interleave over heads).
//
// With ROPE the block also does rope_cache_kernel's work for its head (one kernel instead of two):
// it rotates its query head from the projection q itself (the same operations, so qs holds the same
// values), and the block whose chunk holds position *pos rotates the key head and writes it and the
// value head into the caches before it reads them (blocks of query heads sharing a key head write
// the same values).  qf is then unused.
struct RopeArgs {
    const uint16_t *q, *k, *v;
    const float *cs, *sn;
    uint16_t *kt, *vc;
    int ldq, ldk, ldv;
};

template <int HD, bool ROPE>
__global__ __launch_bounds__(256) void attn_part_kernel(const float* __restrict__ qf, const uint16_t* __restrict__ kt,
                                                        const uint16_t* __restrict__ vc, const int64_t* __restrict__ pos,
                                                        float* __restrict__ part, int H, int Hkv, int L, float sdiv,
                                                        RopeArgs ra) {
    constexpr int Q = HD / 4, G = 256 / HD, HALF = HD / 2;
    __shared__ float qs[HD], dots[4][64], e[64], oacc[256];
    const int bh = blockIdx.x, j = blockIdx.y, S = gridDim.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b = bh / H, h = bh - b * H, kh = h / (H / Hkv);
    const size_t hb = (size_t)b * Hkv + kh;
    const int64_t p = *pos;
    const int n = (int)min((int64_t)L, max((int64_t)0, p + 1));
    const int chunk = (n + S - 1) / S, t0 = min(n, j * chunk), cnt = min(n, t0 + chunk) - t0;
    if constexpr (ROPE) {
        if (tid < HALF) {
            const float c = ra.cs[tid], sv = ra.sn[tid];
            const uint16_t* src = ra.q + (size_t)b * ra.ldq + (size_t)h * HD;
            const float x1 = bf(src[tid]), x2 = bf(src[tid + HALF]);
            qs[tid] = bf(to_bf(sub_rn(mul_rn(x1, c), mul_rn(x2, sv))));
            qs[tid + HALF] = bf(to_bf(add_rn(mul_rn(x2, c), mul_rn(x1, sv))));
            if (p >= t0 && p < t0 + cnt) {
                const uint16_t* ks = ra.k + (size_t)b * ra.ldk + (size_t)kh * HD;
                const float y1 = bf(ks[tid]), y2 = bf(ks[tid + HALF]);
                ra.kt[(hb * HD + tid) * L + p] = to_bf(sub_rn(mul_rn(y1, c), mul_rn(y2, sv)));
                ra.kt[(hb * HD + tid + HALF) * L + p] = to_bf(add_rn(mul_rn(y2, c), mul_rn(y1, sv)));
                const uint16_t* vs = ra.v + (size_t)b * ra.ldv + (size_t)kh * HD;
                ra.vc[(hb * L + p) * HD + tid] = vs[tid];
                ra.vc[(hb * L + p) * HD + tid + HALF] = vs[tid + HALF];
            }
        }
    } else {
        if (tid < HD) qs[tid] = qf[(size_t)bh * HD + tid];
    }
    __syncthreads();
    if (lane < cnt) {
        const uint16_t* kp = kt + (hb * HD + w * Q) * L + t0 + lane;
        float kv[Q];
#pragma unroll
        for (int i = 0; i < Q; ++i) kv[i] = bf(kp[(size_t)i * L]);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < Q; ++i) dot = fmaf(qs[w * Q + i], kv[i], dot);
        dots[w][lane] = dot;
    }
    __syncthreads();
    float m = -INFINITY, l = 0.f;
    if (w == 0) {
        const float sv = lane < cnt ? __fdiv_rn(add_rn(add_rn(dots[0][lane], dots[1][lane]),
                                                          add_rn(dots[2][lane], dots[3][lane])), sdiv)
                                    : -INFINITY;
        m = wave_max(sv);
        const float ev = lane < cnt ? expf(sub_rn(sv, m)) : 0.f;
        e[lane] = ev;
        l = wave_sum(ev);
    }
    __syncthreads();
    // o: G groups of HD threads; group g sums positions g, g + G, ... (loads independent of the sums)
    const int g = tid / HD, i = tid - g * HD;
    const uint16_t* vp = vc + (hb * L + t0) * HD + i;
    float acc = 0.f;
#pragma unroll 8
    for (int t = g; t < cnt; t += G) acc = fmaf(e[t], bf(vp[(size_t)t * HD]), acc);
    oacc[tid] = acc;
    __syncthreads();
    float* out = part + ((size_t)bh * S + j) * (HD + 2);
    if (tid < HD) {
        float o = oacc[tid];
#pragma unroll
        for (int gg = 1; gg < G; ++gg) o = add_rn(o, oacc[gg * HD + tid]);
        out[2 + tid] = o;
    }
    if (tid == 0) {
        out[0] = cnt > 0 ? m : -INFINITY;
        out[1] = l;
    }
}

// Combines the chunks: o[i] = sum_j o_j[i] e^(m_j - M) / sum_j l_j e^(m_j - M), M = max_j m_j,
// rounded to bf16 into out [B, H * hd] (the layout o_proj reads).  Block bh, 256 threads: the
// chunks' (m, l) pairs are staged in LDS with one load each, then thread i < hd adds its column.
// The same chunk partials for head dimension 128 with 16-byte cache loads (cache length L % 8 == 0,
// chunks of a multiple of 8 positions, so every 8-position group starts 16-byte aligned and groups
// past the chunk are not read).  Keys: thread (dim group dd = tid >> 3, position group pg = tid & 7)
// loads dims 4 dd .. 4 dd + 3 of positions 8 pg .. 8 pg + 7 (four 16-byte loads) and forms their
// partial dot products; the 32 dim groups are added with shuffles inside a wave, then across the 4
// waves in LDS.  Values: thread (dims 8 (tid & 15) .. + 7, positions (tid >> 4) + 16 u, u < 4) adds
// e_t v_t over its positions (four 16-byte loads), then the 16 position groups are added the same
// way.  Same partial layout and rotary handling as attn_part_kernel; the sums run in another order.
template <bool ROPE>
__global__ __launch_bounds__(256) void attn_part16_kernel(const float* __restrict__ qf, const uint16_t* __restrict__ kt,
                                                          const uint16_t* __restrict__ vc, const int64_t* __restrict__ pos,
                                                          float* __restrict__ part, int H, int Hkv, int L, float sdiv,
                                                          RopeArgs ra) {
    constexpr int HD = 128, HALF = 64;
    __shared__ float qs[HD], kred[4][64], e[64], vred[4][HD];
    const int bh = blockIdx.x, j = blockIdx.y, S = gridDim.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int b = bh / H, h = bh - b * H, kh = h / (H / Hkv);
    const size_t hb = (size_t)b * Hkv + kh;
    const int64_t p = *pos;
    const int n = (int)min((int64_t)L, max((int64_t)0, p + 1));
    const int chunk = ((n + S - 1) / S + 7) & ~7, t0 = min(n, j * chunk), cnt = min(n, t0 + chunk) - t0;
    if constexpr (ROPE) {
        if (tid < HALF) {
            const float c = ra.cs[tid], sv = ra.sn[tid];
            const uint16_t* src = ra.q + (size_t)b * ra.ldq + (size_t)h * HD;
            const float x1 = bf(src[tid]), x2 = bf(src[tid + HALF]);
            qs[tid] = bf(to_bf(sub_rn(mul_rn(x1, c), mul_rn(x2, sv))));
            qs[tid + HALF] = bf(to_bf(add_rn(mul_rn(x2, c), mul_rn(x1, sv))));
            if (p >= t0 && p < t0 + cnt) {
                const uint16_t* ks = ra.k + (size_t)b * ra.ldk + (size_t)kh * HD;
                const float y1 = bf(ks[tid]), y2 = bf(ks[tid + HALF]);
                ra.kt[(hb * HD + tid) * L + p] = to_bf(sub_rn(mul_rn(y1, c), mul_rn(y2, sv)));
                ra.kt[(hb * HD + tid + HALF) * L + p] = to_bf(add_rn(mul_rn(y2, c), mul_rn(y1, sv)));
                const uint16_t* vs = ra.v + (size_t)b * ra.ldv + (size_t)kh * HD;
                ra.vc[(hb * L + p) * HD + tid] = vs[tid];
                ra.vc[(hb * L + p) * HD + tid + HALF] = vs[tid + HALF];
            }
        }
    } else {
        if (tid < HD) qs[tid] = qf[(size_t)bh * HD + tid];
    }
    __syncthreads();
    // keys: 8 positions x 4 dims per thread
    const int pg = tid & 7, dd = tid >> 3;
    float dot[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (8 * pg < cnt) {
        uint4 kv[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) kv[d] = *(const uint4*)(kt + (hb * HD + 4 * dd + d) * L + t0 + 8 * pg);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const float qd = qs[4 * dd + d];
            const uint32_t wv[4] = {kv[d].x, kv[d].y, kv[d].z, kv[d].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                dot[2 * u] = fmaf(qd, __uint_as_float(wv[u] << 16), dot[2 * u]);
                dot[2 * u + 1] = fmaf(qd, __uint_as_float(wv[u] & 0xFFFF0000u), dot[2 * u + 1]);
            }
        }
    }
    // add the 8 dim groups of this wave (lanes 8 apart), then the 4 waves in LDS
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        float v = dot[u];
        v = add_rn(v, __shfl_xor(v, 8));
        v = add_rn(v, __shfl_xor(v, 16));
        v = add_rn(v, __shfl_xor(v, 32));
        dot[u] = v;
    }
    if (lane < 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) kred[w][8 * lane + u] = dot[u];
    }
    __syncthreads();
    float m = -INFINITY, l = 0.f;
    if (w == 0) {
        const float sv = lane < cnt ? __fdiv_rn(add_rn(add_rn(kred[0][lane], kred[1][lane]),
                                                          add_rn(kred[2][lane], kred[3][lane])), sdiv)
                                    : -INFINITY;
        m = wave_max(sv);
        const float ev = lane < cnt ? expf(sub_rn(sv, m)) : 0.f;
        e[lane] = ev;
        l = wave_sum(ev);
    }
    __syncthreads();
    // values: 8 dims x 4 positions per thread
    const int dg = tid & 15, pp = tid >> 4;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    uint4 vv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int t = pp + 16 * u;
        vv[u] = t < cnt ? *(const uint4*)(vc + (hb * L + t0 + t) * HD + 8 * dg) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int t = pp + 16 * u;
        const float et = t < cnt ? e[t] : 0.f;
        const uint32_t wv[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            acc[2 * c] = fmaf(et, __uint_as_float(wv[c] << 16), acc[2 * c]);
            acc[2 * c + 1] = fmaf(et, __uint_as_float(wv[c] & 0xFFFF0000u), acc[2 * c + 1]);
        }
    }
    // add the 4 position groups of this wave (lanes 16 apart), then the 4 waves in LDS
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        float v = acc[c];
        v = add_rn(v, __shfl_xor(v, 16));
        v = add_rn(v, __shfl_xor(v, 32));
        acc[c] = v;
    }
    if (lane < 16) {
#pragma unroll
        for (int c = 0; c < 8; ++c) vred[w][8 * lane + c] = acc[c];
    }
    __syncthreads();
    float* dst = part + ((size_t)bh * S + j) * (HD + 2);
    if (tid < HD) dst[2 + tid] = add_rn(add_rn(vred[0][tid], vred[1][tid]), add_rn(vred[2][tid], vred[3][tid]));
    if (tid == 0) {
        dst[0] = cnt > 0 ? m : -INFINITY;
        dst[1] = l;
    }
}

__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part, uint16_t* __restrict__ out,
                                                           int hd, int S) {
    __shared__ float mj[256], fj[256], red[4];
    const int bh = blockIdx.x, tid = threadIdx.x;
    const float* p = part + (size_t)bh * S * (hd + 2);
    const float mv = tid < S ? p[(size_t)tid * (hd + 2)] : -INFINITY;
    const float lv = tid < S ? p[(size_t)tid * (hd + 2) + 1] : 0.f;
    const float M = block_max(mv, red);
    const float f = mv == -INFINITY ? 0.f : expf(sub_rn(mv, M));
    mj[tid] = lv;
    fj[tid] = f;
    __syncthreads();
    if (tid < hd) {
        float num = 0.f, den = 0.f;
        for (int j = 0; j < S; ++j) {
            num = fmaf(p[(size_t)j * (hd + 2) + 2 + tid], fj[j], num);
            den = fmaf(mj[j], fj[j], den);
        }
        out[(size_t)bh * hd + tid] = to_bf(__fdiv_rn(num, den));
    }
}

// out = bf16(bf16(silu(g)) * u), silu(x) = x / (1 + exp(-x)) in fp32 (F.silu then the product of
// MLP.forward), over rows of n elements: row r of g / u starts ld elements after row r - 1 (the
// two halves of one fused projection), out is [rows, n].
// Vector form: n % 8 == 0, ld % 8 == 0, 16-byte aligned rows; block (chunk of 256 x 8 elements, row).
__global__ __launch_bounds__(256) void silu_mul8_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                        uint16_t* __restrict__ out, int n, int64_t ld) {
    const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (c >= n) return;
    const size_t r = blockIdx.y, i = r * ld + c;
    const uint4 ga = *(const uint4*)(g + i), ua = *(const uint4*)(u + i);
    const uint16_t* gs = (const uint16_t*)&ga;
    const uint16_t* us = (const uint16_t*)&ua;
    uint4 oa;
    uint16_t* os = (uint16_t*)&oa;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float x = bf(gs[j]);
        const float sv = bf(to_bf(__fdiv_rn(x, add_rn(1.f, expf(-x)))));
        os[j] = to_bf(mul_rn(sv, bf(us[j])));
    }
    *(uint4*)(out + r * n + c) = oa;
}

__global__ void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                uint16_t* __restrict__ out, int rows, int n, int64_t ld) {
    const int64_t total = (int64_t)rows * n;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / n, i = r * ld + (e - r * n);
        const float x = bf(g[i]);
        const float sv = bf(to_bf(__fdiv_rn(x, add_rn(1.f, expf(-x)))));
        out[e] = to_bf(mul_rn(sv, bf(u[i])));
    }
}

typedef __bf16 hbf16x8 __attribute__((ext_vector_type(8)));
typedef float hf32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 head_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Tied output head of the decode step: y[b, v] = sum_k float(x[b, k]) * float(w[v, k]) with fp32
// accumulation, x the normed hidden state (bf16 [NB, K], NB <= 16) and w the bf16 embedding [V, K]
// -- the products of Llama._head's F.linear(x.float(), embedding.float()), read from the bf16
// embedding itself instead of an fp32 copy of it.  v_mfma_f32_16x16x32_bf16 forms the same
// products (bf16 x bf16 is exact in fp32) and sums them in fp32 in its own order.  Block: 32
// embedding rows (two 16-row tiles) and 4 waves splitting K; lane l takes x row l & 15 and row l & 15
// of each tile at k = 8 (l >> 4) .. + 7 of every 32-wide step (16-byte loads, the MFMA operands as
// loaded; rows past NB or V read zeros through the buffer resources).  D steps of loads in flight
// per wave, issued unconditionally (past the wave's range they read zeros), so the loop has no
// branch for the compiler to wait at.  Requires K % (128 D) == 0.
template <int D>
__global__ __launch_bounds__(256) void head_mfma_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                        float* __restrict__ y, int NB, int V, int K) {
    __shared__ hf32x4 red[4][2][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * 32, rows = min(32, V - n0);
    const int kw = K / 4, nst = kw / 32;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, NB * K * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(w + (size_t)n0 * K), (short)0, rows * K * 2, 0x00020000);
    const uint32_t base = ((uint32_t)j * (uint32_t)K + (uint32_t)(wave * kw + q * 8)) * 2u;
    const uint32_t tile1 = 16u * (uint32_t)K * 2u;
    uint4 xa[D], wa[D], wb[D];
    auto issue = [&](int d, int st) {
        const uint32_t off = st < nst ? base + (uint32_t)st * 64u : 0x80000000u;
        xa[d] = head_load(xr, off);
        wa[d] = head_load(wr, off);
        wb[d] = head_load(wr, st < nst ? off + tile1 : 0x80000000u);
    };
    hf32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    for (int st = 0; st < nst; st += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const hbf16x8 a = __builtin_bit_cast(hbf16x8, xa[d]);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(hbf16x8, wa[d]), acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(hbf16x8, wb[d]), acc1, 0, 0, 0);
            issue(d, st + d + D);
        }
    }
    // Lane l holds x rows 4 (l >> 4) + r of embedding row l & 15 of each tile; the waves' K ranges
    // are added in order in LDS.
    red[wave][0][lane] = acc0;
    red[wave][1][lane] = acc1;
    __syncthreads();
    if (wave >= 2) return;
    hf32x4 tot = red[0][wave][lane];
#pragma unroll
    for (int v = 1; v < 4; ++v) tot += red[v][wave][lane];
    const int n = n0 + wave * 16 + j;
    if (n >= V) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * q + r;
        if (m < NB) y[(size_t)m * V + n] = tot[r];
    }
}

// Causal attention of the prefill (Attention.attend: softmax((q . k) / sqrt(hd), key <= query) times
// v, for the T query positions start .. start + T - 1 over cache positions 0 .. start + T - 1) as one
// flash-attention kernel, hd = 128.  Block (query tile of 64 rows, head, batch), 4 waves of 16 rows;
// per step of 64 cache positions the key tile is staged in LDS as [position][dim] and the value tile
// as [dim][position] (the caches hold them the other way round for the decoding kernels), then per
// wave, with v_mfma_f32_16x16x32_bf16:
//   S^T = K Q^T   (A: 16 positions x 8 dims per lane from LDS; B: the wave's q rows, in registers),
//   O^T += V^T P^T (A: 16 dims x 8 positions per lane from LDS; B: P^T straight from S^T's lanes).
// Lane l ends S^T holding positions 16 mt + 4 (l >> 4) + r of query row l & 15, so P^T needs no
// shuffle: the O^T product takes its 32 positions per step in that order (the same order on both
// operands, so the sum is unchanged), and O^T lands with query row l & 15 in the lane that holds
// that row's softmax statistics.  bf16 x bf16 products are exact and summed in fp32, as the bf16
// score product with fp32 output; P (fp32) enters the value product as bf16 hi + lo (2^-18 relative),
// the values being bf16; the running max / sum rescale as in any online softmax.  Positions past
// the written ones read as zeros (the cache may hold anything there) and are masked with -inf.
constexpr int FA_KP = 136;   // key tile row pitch in elements: 128 dims + 8
constexpr int FA_VP = 72;    // value tile row pitch: 64 positions + 8
__global__ __launch_bounds__(256) void attn_prefill_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kt,
                                                           const uint16_t* __restrict__ vc, uint16_t* __restrict__ out,
                                                           int start, int T, int H, int Hkv, int Lc, int ldo, float scale) {
    __shared__ __align__(16) uint16_t ks[64 * FA_KP];
    __shared__ __align__(16) uint16_t vt[128 * FA_VP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, g = lane >> 4;
    const int nT = (T + 63) / 64, tile = nT - 1 - (int)blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t0 = tile * 64, row = t0 + 16 * wave + j, qp = start + row;
    const int kmax = start + min(t0 + 63, T - 1);             // last position the tile's rows see
    const size_t hb = (size_t)b * Hkv + h / (H / Hkv);
    hbf16x8 qb[4];
    const uint16_t* qrow = q + (((size_t)b * H + h) * T + min(row, T - 1)) * 128;
#pragma unroll
    for (int k = 0; k < 4; ++k) qb[k] = __builtin_bit_cast(hbf16x8, *(const uint4*)(qrow + 32 * k + 8 * g));
    float m_run = -INFINITY, l_run = 0.f;
    hf32x4 o[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] = hf32x4{0.f, 0.f, 0.f, 0.f};
    const int nk = kmax / 64 + 1;
    // Tile rows for the LDS staging: keys as (dims 4 kdg .. + 3, positions 8 kpg .. + 7), values as
    // (positions 4 vpg .. + 3, dims 8 vdg .. + 7); the next step's rows load while this one computes.
    const int kdg = tid & 31, kpg = tid >> 5, vdg = tid & 15, vpg = tid >> 4;
    uint4 kr[4], vr[4];
    auto load = [&](int p0) {
        const int p = p0 + 8 * kpg;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            kr[r] = p <= kmax ? *(const uint4*)(kt + (hb * 128 + 4 * kdg + r) * Lc + p) : uint4{0u, 0u, 0u, 0u};
            const int pp = p0 + 4 * vpg + r;
            vr[r] = pp <= kmax ? *(const uint4*)(vc + (hb * Lc + pp) * 128 + 8 * vdg) : uint4{0u, 0u, 0u, 0u};
        }
    };
    load(0);
    for (int kb = 0; kb < nk; ++kb) {
        const int p0 = kb * 64;
        __syncthreads();                                      // the previous step's tiles are read
        {
            const uint16_t* rs = (const uint16_t*)kr;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                alignas(8) uint16_t w[4] = {rs[i], rs[8 + i], rs[16 + i], rs[24 + i]};
                *(uint2*)(ks + (8 * kpg + i) * FA_KP + 4 * kdg) = *(const uint2*)w;
            }
            const uint16_t* vs = (const uint16_t*)vr;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                alignas(8) uint16_t w[4] = {vs[i], vs[8 + i], vs[16 + i], vs[24 + i]};
                *(uint2*)(vt + (8 * vdg + i) * FA_VP + 4 * vpg) = *(const uint2*)w;
            }
        }
        __syncthreads();
        if (kb + 1 < nk) load(p0 + 64);
        hf32x4 sc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            sc[mt] = hf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    *(const hbf16x8*)(ks + (16 * mt + j) * FA_KP + 32 * k + 8 * g), qb[k], sc[mt], 0, 0, 0);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = mul_rn(sc[mt][r], scale);
                sc[mt][r] = p0 + 16 * mt + 4 * g + r > qp ? -INFINITY : v;
                mx = fmaxf(mx, sc[mt][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);                 // finite: position 0 is in every row's first step
        const float alpha = expf(sub_rn(m_run, m_new));
        float ps = 0.f;
        alignas(16) uint16_t hi[2][8], lo[2][8];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = expf(sub_rn(sc[mt][r], m_new));
                ps = add_rn(ps, pv);
                const uint16_t ph = to_bf(pv);
                hi[mt >> 1][(mt & 1) * 4 + r] = ph;
                lo[mt >> 1][(mt & 1) * 4 + r] = to_bf(sub_rn(pv, bf(ph)));
            }
        ps = add_rn(ps, __shfl_xor(ps, 16));
        ps = add_rn(ps, __shfl_xor(ps, 32));
        l_run = add_rn(mul_rn(l_run, alpha), ps);
        m_run = m_new;
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) o[mt] *= alpha;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const hbf16x8 bh = __builtin_bit_cast(hbf16x8, *(const uint4*)hi[k]);
            const hbf16x8 bl = __builtin_bit_cast(hbf16x8, *(const uint4*)lo[k]);
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                const uint16_t* vr = vt + (16 * mt + j) * FA_VP + 32 * k + 4 * g;
                const uint2 a0 = *(const uint2*)vr, a1 = *(const uint2*)(vr + 16);
                const hbf16x8 a = __builtin_bit_cast(hbf16x8, uint4{a0.x, a0.y, a1.x, a1.y});
                o[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, o[mt], 0, 0, 0);
                o[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, o[mt], 0, 0, 0);
            }
        }
    }
    if (row >= T) return;
    uint16_t* orow = out + ((size_t)b * T + row) * ldo + (size_t)h * 128;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
        alignas(8) uint16_t w[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = to_bf(__fdiv_rn(o[mt][r], l_run));
        *(uint2*)(orow + 16 * mt + 4 * g) = *(const uint2*)w;
    }
}

// Start of a decode step (Llama.decode_step's embedding lookup and rotary angles): block b < B copies
// embedding row tok[b] (bf16 [V, d]) into x[b] (a token outside 0..V-1 gives a zero row); block B
// computes the angles pos * inv[i] in fp32 and their cosine and sine, as pos.float() * inv, .cos()
// and .sin() do.
__global__ __launch_bounds__(256) void step_in_kernel(const int64_t* __restrict__ tok, const int64_t* __restrict__ pos,
                                                      const float* __restrict__ inv, const uint16_t* __restrict__ emb,
                                                      uint16_t* __restrict__ x, float* __restrict__ cs,
                                                      float* __restrict__ sn, int B, int d, int half, int V) {
    const int b = blockIdx.x, tid = threadIdx.x;
    if (b == B) {
        const float pf = (float)*pos;
        for (int i = tid; i < half; i += 256) {
            const float a = mul_rn(pf, inv[i]);
            cs[i] = cosf(a);
            sn[i] = sinf(a);
        }
        return;
    }
    const int64_t t = tok[b];
    const bool ok = t >= 0 && t < V;
    const uint4* src = (const uint4*)(emb + (ok ? (size_t)t * d : 0));
    uint4* dst = (uint4*)(x + (size_t)b * d);
    for (int i = tid; i < d / 8; i += 256) dst[i] = ok ? src[i] : make_uint4(0, 0, 0, 0);
}

// (value, index) order of torch.argmax: NaN above everything, then larger values, then the lower
// index.
__device__ __forceinline__ bool am_better(float a, int ia, float b, int ib) {
    const bool na = a != a, nb = b != b;
    if (na != nb) return na;
    if (!na && a != b) return a > b;
    return ia < ib;
}

// End of a decode step (greedy(), tok.copy_ and pos.add_(1)): block b writes into tok[b] the index
// of the first maximum of logits row b (V values, rows ld apart); block 0 then advances pos.
__global__ __launch_bounds__(1024) void step_out_kernel(const float* __restrict__ logits, int V, int64_t ld,
                                                        int64_t* __restrict__ tok, int64_t* __restrict__ pos) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* row = logits + (size_t)b * ld;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    auto take = [&](float v, int i) {
        if (am_better(v, i, best, idx)) {
            best = v;
            idx = i;
        }
    };
    if ((V & 3) == 0 && ((uintptr_t)row & 15) == 0) {
        // 16-byte loads, 8 per thread in flight before any comparison (the values of a row are
        // independent: a loop that compares each load before issuing the next waits once per load)
        const float4* r4 = (const float4*)row;
        const int n4 = V / 4;
        for (int base = 0; base < n4; base += 8 * 1024) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i4 = base + u * 1024 + tid;
                v[u] = i4 < n4 ? r4[i4] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = 4 * (base + u * 1024 + tid);
                if (i < V) {
                    take(v[u].x, i);
                    take(v[u].y, i + 1);
                    take(v[u].z, i + 2);
                    take(v[u].w, i + 3);
                }
            }
        }
    } else {
        for (int i = tid; i < V; i += 1024) take(row[i], i);
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(idx, off);
        if (am_better(ov, oi, best, idx)) {
            best = ov;
            idx = oi;
        }
    }
    if (lane == 0) {
        bv[w] = best;
        bi[w] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int j = 1; j < 16; ++j)
            if (am_better(bv[j], bi[j], best, idx)) {
                best = bv[j];
                idx = bi[j];
            }
        tok[b] = idx;
        if (b == 0) *pos += 1;
    }
}

int launched() { return (int)hipGetLastError(); }

}  // namespace

extern "C" {

// Error codes: 0, a hipError_t, or -1 for arguments these kernels do not take.
int tfp8_llm_add_rmsnorm(const void* x, const void* r, void* h, void* y, const void* w, int rows, int d, float eps,
                         void* stream) {
    if (rows < 0 || d <= 0 || d % 8 || d > 2048 * 4 || !x || !y || !w || (r && !h)) return -1;
    if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)w | (uintptr_t)r | (uintptr_t)h) % 16) return -1;
    if (rows == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    const uint16_t *xp = (const uint16_t*)x, *rp = (const uint16_t*)r, *wp = (const uint16_t*)w;
    uint16_t *hp = (uint16_t*)h, *yp = (uint16_t*)y;
    if (d <= 2048) add_rmsnorm_kernel<1><<<rows, 256, 0, s>>>(xp, rp, hp, yp, wp, d, eps);
    else if (d <= 4096) add_rmsnorm_kernel<2><<<rows, 256, 0, s>>>(xp, rp, hp, yp, wp, d, eps);
    else add_rmsnorm_kernel<4><<<rows, 256, 0, s>>>(xp, rp, hp, yp, wp, d, eps);
    return launched();
}

// Row strides ldq >= H hd, ldk and ldv >= Hkv hd (elements).
int tfp8_llm_rope_cache(const void* q, const void* k, const void* v, const float* cs, const float* sn, float* qf,
                        void* kt, void* vc, const int64_t* pos, int B, int H, int Hkv, int hd, int L, int ldq,
                        int ldk, int ldv, void* stream) {
    if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || hd % 2 || hd > 512 || L <= 0) return -1;
    if (ldq < H * hd || ldk < Hkv * hd || ldv < Hkv * hd) return -1;
    if (!q || !k || !v || !cs || !sn || !qf || !kt || !vc || !pos) return -1;
    if (B == 0) return 0;
    rope_cache_kernel<<<dim3(H + Hkv, B), hd / 2, 0, (hipStream_t)stream>>>(
        (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, cs, sn, qf, (uint16_t*)kt, (uint16_t*)vc, pos, H,
        Hkv, hd, L, ldq, ldk,
        ldv);
    return launched();
}

// Chunks S with S * 64 >= L and S <= 256; head dimension 64 or 128; part holds B * H * S * (hd + 2) floats.
int tfp8_llm_attention(const float* qf, const void* kt, const void* vc, const int64_t* pos, float* part, int S,
                       void* out, int B, int H, int Hkv, int hd, int L, float sdiv, void* stream) {
    if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv || (hd != 64 && hd != 128) || L <= 0) return -1;
    if (S <= 0 || (int64_t)S * 64 < L || S > 256 || !qf || !kt || !vc || !pos || !part || !out) return -1;
    if (B == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    const uint16_t *kp = (const uint16_t*)kt, *vp = (const uint16_t*)vc;
    const RopeArgs none{};
    const bool v16 = hd == 128 && L % 8 == 0 && ((uintptr_t)kt | (uintptr_t)vc) % 16 == 0;
    if (v16) attn_part16_kernel<false><<<dim3(B * H, S), 256, 0, s>>>(qf, kp, vp, pos, part, H, Hkv, L, sdiv, none);
    else if (hd == 128) attn_part_kernel<128, false><<<dim3(B * H, S), 256, 0, s>>>(qf, kp, vp, pos, part, H, Hkv, L, sdiv, none);
    else attn_part_kernel<64, false><<<dim3(B * H, S), 256, 0, s>>>(qf, kp, vp, pos, part, H, Hkv, L, sdiv, none);
    int rc = launched();
    if (rc) return rc;
    attn_combine_kernel<<<B * H, 256, 0, s>>>(part, (uint16_t*)out, hd, S);
    return launched();
}

// Rows of q / k / v: B * T, row r = b * T + t, ldq / ldk / ldv elements apart; 0 <= start and
// start + T <= L; hd even and at most 256 (the key tile takes hd * (RP_T + 2) * 2 bytes of LDS).
int tfp8_llm_rope_prefill(const void* q, const void* k, const void* v, const float* cs, const float* sn, void* qo,
                          void* kt, void* vc, int start, int B, int T, int H, int Hkv, int hd, int L, int ldq, int ldk,
                          int ldv, void* stream) {
    if (B < 0 || T < 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd <= 0 || hd % 2 || hd > 256 || L <= 0) return -1;
    if (start < 0 || (int64_t)start + T > L || ldq < H * hd || ldk < Hkv * hd || ldv < Hkv * hd) return -1;
    if (!q || !k || !v || !cs || !sn || !qo || !kt || !vc) return -1;
    if (B == 0 || T == 0) return 0;
    const int64_t tiles = (int64_t)B * ((T + RP_T - 1) / RP_T);
    if (tiles > 65535) return -1;                             // gridDim.y
    const dim3 grid(H + Hkv, (unsigned)tiles);
    const size_t lds = (size_t)hd * (RP_T + 2) * 2;
    // 4 dims a thread where every row and the cos / sin rows allow 8- / 16-byte accesses
    const bool v4 = hd % 8 == 0 && ldq % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && L % 4 == 0 &&
                    ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)qo | (uintptr_t)vc) % 8 == 0 &&
                    ((uintptr_t)cs | (uintptr_t)sn) % 16 == 0;
    if (v4)
        rope_prefill_kernel<4><<<grid, 256, lds, (hipStream_t)stream>>>(
            (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, cs, sn, (uint16_t*)qo, (uint16_t*)kt,
            (uint16_t*)vc, start, T, H, Hkv, hd, L, ldq, ldk, ldv);
    else
        rope_prefill_kernel<1><<<grid, 256, lds, (hipStream_t)stream>>>(
            (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, cs, sn, (uint16_t*)qo, (uint16_t*)kt,
            (uint16_t*)vc, start, T, H, Hkv, hd, L, ldq, ldk, ldv);
    return launched();
}

// tfp8_llm_rope_cache followed by tfp8_llm_attention in two kernels instead of three: the same
// cache contents and the same output bits (no qf buffer).  Arguments as there; a position outside
// the cache is refused on the host by the caller, as for rope_cache.
int tfp8_llm_rope_attention(const void* q, const void* k, const void* v, const float* cs, const float* sn, void* kt,
                            void* vc, const int64_t* pos, float* part, int S, void* out, int B, int H, int Hkv, int hd,
                            int L, int ldq, int ldk, int ldv, float sdiv, void* stream) {
    if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv || (hd != 64 && hd != 128) || L <= 0) return -1;
    if (S <= 0 || (int64_t)S * 64 < L || S > 256 || !kt || !vc || !pos || !part || !out) return -1;
    if (ldq < H * hd || ldk < Hkv * hd || ldv < Hkv * hd || !q || !k || !v || !cs || !sn) return -1;
    if (B == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    const RopeArgs ra{(const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, cs, sn, (uint16_t*)kt,
                      (uint16_t*)vc, ldq, ldk, ldv};
    const uint16_t *kp = (const uint16_t*)kt, *vp = (const uint16_t*)vc;
    const bool v16 = hd == 128 && L % 8 == 0 && ((uintptr_t)kt | (uintptr_t)vc) % 16 == 0;
    if (v16) attn_part16_kernel<true><<<dim3(B * H, S), 256, 0, s>>>(nullptr, kp, vp, pos, part, H, Hkv, L, sdiv, ra);
    else if (hd == 128) attn_part_kernel<128, true><<<dim3(B * H, S), 256, 0, s>>>(nullptr, kp, vp, pos, part, H, Hkv, L, sdiv, ra);
    else attn_part_kernel<64, true><<<dim3(B * H, S), 256, 0, s>>>(nullptr, kp, vp, pos, part, H, Hkv, L, sdiv, ra);
    int rc = launched();
    if (rc) return rc;
    attn_combine_kernel<<<B * H, 256, 0, s>>>(part, (uint16_t*)out, hd, S);
    return launched();
}

// rows x n elements, input row stride ld >= n.
int tfp8_llm_silu_mul(const void* g, const void* u, void* out, int rows, int n, int64_t ld, void* stream) {
    if (rows < 0 || n < 0 || ld < n || !g || !u || !out) return -1;
    if (rows == 0 || n == 0) return 0;
    // 8 elements a thread for many rows (prefill); a decoding step's few rows keep one element a thread,
    // whose more threads finish sooner than a few blocks each evaluating 8 exp / divide in a row.
    if (rows >= 64 && rows <= 65535 && n % 8 == 0 && ld % 8 == 0 &&
        ((uintptr_t)g | (uintptr_t)u | (uintptr_t)out) % 16 == 0) {
        silu_mul8_kernel<<<dim3((unsigned)((n / 8 + 255) / 256), (unsigned)rows), 256, 0, (hipStream_t)stream>>>(
            (const uint16_t*)g, (const uint16_t*)u, (uint16_t*)out, n, ld);
        return launched();
    }
    const int64_t blocks = ((int64_t)rows * n + 255) / 256;
    silu_mul_kernel<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)g, (const uint16_t*)u, (uint16_t*)out, rows, n, ld);
    return launched();
}


// q bf16 [B, H, T, 128] contiguous, caches kt [B, Hkv, 128, Lc] / vc [B, Hkv, Lc, 128] (Lc % 8 == 0),
// out bf16 rows b * T + t of ldo elements (ldo % 4 == 0, >= H * 128); 16-byte aligned pointers.
int tfp8_llm_attn_prefill(const void* q, const void* kt, const void* vc, void* out, int start, int B, int T, int H,
                          int Hkv, int hd, int Lc, int ldo, float scale, void* stream) {
    if (B < 0 || T < 0 || H <= 0 || Hkv <= 0 || H % Hkv || hd != 128 || Lc <= 0 || Lc % 8) return -1;
    if (start < 0 || (int64_t)start + T > Lc || ldo < H * 128 || ldo % 4 || !q || !kt || !vc || !out) return -1;
    if (((uintptr_t)q | (uintptr_t)kt | (uintptr_t)vc | (uintptr_t)out) % 16) return -1;
    if (B == 0 || T == 0) return 0;
    if (B > 65535 || H > 65535) return -1;
    attn_prefill_kernel<<<dim3((unsigned)((T + 63) / 64), (unsigned)H, (unsigned)B), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)q, (const uint16_t*)kt, (const uint16_t*)vc, (uint16_t*)out, start, T, H, Hkv, Lc, ldo, scale);
    return launched();
}

// rows <= 16, K % 512 == 0, V * K * 2 < 2^31.
int tfp8_llm_head(const void* x, const void* w, float* y, int rows, int V, int K, void* stream) {
    if (rows < 0 || rows > 16 || V < 0 || K <= 0 || K % 512 || !x || !w || !y) return -1;
    if ((int64_t)V * K * 2 >= (1LL << 31)) return -1;
    if (((uintptr_t)x | (uintptr_t)w) % 16) return -1;
    if (rows == 0 || V == 0) return 0;
    head_mfma_kernel<4><<<(unsigned)((V + 31) / 32), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)x, (const uint16_t*)w, y, rows, V, K);
    return launched();
}

// tok / pos int64 on the device, inv fp32 [half], emb bf16 [V, d] (d % 8 == 0, 16-byte aligned), x bf16
// [B, d], cs / sn fp32 [half].
int tfp8_llm_step_in(const int64_t* tok, const int64_t* pos, const float* inv, const void* emb, void* x, float* cs,
                     float* sn, int B, int d, int half, int V, void* stream) {
    if (B < 0 || d <= 0 || d % 8 || half <= 0 || V <= 0 || !tok || !pos || !inv || !emb || !x || !cs || !sn) return -1;
    if (((uintptr_t)emb | (uintptr_t)x) % 16) return -1;
    step_in_kernel<<<B + 1, 256, 0, (hipStream_t)stream>>>(tok, pos, inv, (const uint16_t*)emb, (uint16_t*)x, cs, sn,
                                                            B, d, half, V);
    return launched();
}

// logits fp32, B rows of V values ld apart; tok int64 [B], pos int64 [1] (advanced by one).
int tfp8_llm_step_out(const float* logits, int B, int V, int64_t ld, int64_t* tok, int64_t* pos, void* stream) {
    if (B <= 0 || V <= 0 || ld < V || !logits || !tok || !pos) return -1;
    step_out_kernel<<<B, 1024, 0, (hipStream_t)stream>>>(logits, V, ld, tok, pos);
    return launched();
}

}  // extern "C"
