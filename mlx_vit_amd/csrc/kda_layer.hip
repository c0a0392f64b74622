// kda_layer.hip -- gfx950 kernels for the two elementwise ends of the
// GatedDeltaLayer around the KDA recurrence, with their adjoints.
//
//   producer (nope_gdn_mlx.py:796-821; ShortCausalConv1d nope_gdn_mlx.py:369-431;
//             l2_normalize / softplus nope_gdn_mlx.py:77-86)
//       q    = l2norm(silu(conv4(xq))) * scale
//       k    = l2norm(silu(conv4(xk)))
//       v    = silu(conv4(xv))
//       g    = -exp(A_log[h]) * softplus(xf + dt_bias)
//       beta = sigmoid(xb) * beta_mult
//     conv4 is the causal depthwise 4-tap convolution with bias:
//     y[t, c] = bias[c] + sum_k w[c, k] x[t + k - 3, c], rows before 0 read as
//     zero.  l2norm runs over the whole H*D row: the reference normalises
//     before it splits the heads (nope_gdn_mlx.py:811-812, 831-833).
//   gated RMSNorm (RMSNormGated, nope_gdn_mlx.py:340-366, 880-885)
//       y = o * rsqrt(mean_d(o^2) + eps) * w * sigmoid(z), per head of D channels.
//
// Layout: a workgroup holds NW = ceil(H*D / 256) waves side by side across the
// channels; lane l of wave w owns channels 256 w + 4 l .. +3, so every row
// access is one 8-byte (bf16) or 16-byte (fp32) load per lane and a whole H*D
// row lives in one workgroup (the l2 norms reduce through LDS).  These kernels
// are HBM- and VALU-bound; nothing here is MFMA-shaped.  Parameter gradients
// are per-workgroup partial sums in the caller's workspace, summed by a
// column-reduction kernel, so every result is deterministic (no atomics).
#include <algorithm>
#include <cstdint>

#include "kda_internal.h"
#include "kda_device.h"

namespace kda {
namespace {

constexpr int KC = 4;        // conv taps (ShortCausalConv1d(kernel_size=4))
constexpr int CPW = 256;     // channels per wave
constexpr int MAXW = 8;      // H*D <= 2048
constexpr int PR = 2;        // producer forward: rows per workgroup
constexpr int BR = 8;        // producer backward: rows per strip
constexpr int BNS = 4;       // producer backward: strips per workgroup
constexpr int NR = 4;        // norm forward: rows per workgroup
constexpr int NRB = 4;       // norm backward: rows per strip
constexpr int NNS = 2;       // norm backward: strips per workgroup
constexpr int NPV = 17;      // producer parameter-gradient values per channel
constexpr float L2_EPS = 1e-12f;

template <typename T> struct Vec4;
template <> struct Vec4<float> {
    static __device__ __forceinline__ void ld(const float* p, float* x) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    }
    static __device__ __forceinline__ void st(float* p, const float* x) {
        *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    }
};
template <> struct Vec4<uint16_t> {
    static __device__ __forceinline__ void ld(const uint16_t* p, float* x) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        x[0] = __uint_as_float(v.x << 16); x[1] = __uint_as_float(v.x & 0xffff0000u);
        x[2] = __uint_as_float(v.y << 16); x[3] = __uint_as_float(v.y & 0xffff0000u);
    }
    static __device__ __forceinline__ void st(uint16_t* p, const float* x) {
        *reinterpret_cast<uint2*>(p) = make_uint2(pack2bf(x[0], x[1]), pack2bf(x[2], x[3]));
    }
};

// log(1 + e^x) without overflow (nope_gdn_mlx.py:83-86): max(x, 0) + log1p(e^-|x|),
// log1p(e) = log(u) - ((u - 1) - e) / u with u = 1 + e (the rounding of u is
// compensated to first order), on the hardware log
__device__ __forceinline__ float softplus(float x) {
    const float e = __expf(-fabsf(x));
    const float u = 1.f + e;
    return fmaxf(x, 0.f) + (__logf(u) - ((u - 1.f) - e) * __builtin_amdgcn_rcpf(u));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}
// Sum over aligned groups of n lanes (n a power of two <= 64).
__device__ __forceinline__ float lanes_sum(float v, int n) {
    for (int m = n >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// Workgroup p runs on XCD p % 8; give each XCD a contiguous range of logical
// workgroups so that neighbouring row strips (which share conv halo rows)
// meet in the same L2.
__device__ __forceinline__ int xcd_remap(int p, int n) {
    const int q = n >> 3, r = n & 7, x = p & 7, j = p >> 3;
    return x * q + min(x, r) + j;
}

struct Lanes {
    int HD, w, lane, NW, cc, h;
    bool live;
    __device__ Lanes(int H, int D) {
        HD = H * D;
        w = threadIdx.x >> 6;
        lane = threadIdx.x & 63;
        NW = blockDim.x >> 6;
        const int c = w * CPW + lane * 4;
        live = c < HD;
        cc = live ? c : 0;   // idle lanes address channel 0; their results are dropped
        h = cc / D;
    }
};

template <int I>
__device__ __forceinline__ void load_taps(const ProdArgs& a, const Lanes& L, float (&wt)[4][KC], float (&bias)[4]) {
    const float4* p = reinterpret_cast<const float4*>(a.conv_w + ((size_t)I * L.HD + L.cc) * KC);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float4 v = p[e];
        wt[e][0] = v.x; wt[e][1] = v.y; wt[e][2] = v.z; wt[e][3] = v.w;
    }
    if (a.conv_b) {
        const float4 v = *reinterpret_cast<const float4*>(a.conv_b + (size_t)I * L.HD + L.cc);
        bias[0] = v.x; bias[1] = v.y; bias[2] = v.z; bias[3] = v.w;
    } else {
        bias[0] = bias[1] = bias[2] = bias[3] = 0.f;
    }
}

// ---------------------------------------------------------------- producer, forward
// Workgroup = (batch row b, strip of PR tokens).
// Conv + SiLU of PR rows of conv input i at channel quad cc (rows before 0
// read as zero, rows past T clamp; their results are dropped by the caller).
// The conv input is a template parameter so that its pointer is a fixed field
// of the kernel arguments (a runtime choice among xq / xk / xv makes the
// compiler copy the argument block to scratch memory).
template <typename ST, int I>
__device__ __forceinline__ void conv_silu_rows(const ProdArgs& a, const Lanes& L, int t0, size_t rb,
                                               float (&out)[PR][4]) {
    const int T = a.T;
    const ST* x = static_cast<const ST*>(I == 0 ? a.xq : I == 1 ? a.xk : a.xv);
    float wt[4][KC], bias[4];
    load_taps<I>(a, L, wt, bias);
    float xr[PR + KC - 1][4];
#pragma unroll
    for (int r = 0; r < PR + KC - 1; ++r) {
        const int t = t0 - (KC - 1) + r;
        Vec4<ST>::ld(x + (rb + min(max(t, 0), T - 1)) * a.ld_x + L.cc, xr[r]);
        if (t < 0) xr[r][0] = xr[r][1] = xr[r][2] = xr[r][3] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < PR; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float y = bias[e];
#pragma unroll
            for (int k = 0; k < KC; ++k) y = fmaf(wt[e][k], xr[j + k][e], y);
            out[j][e] = y * sigm(y);
        }
}

// Workgroup = (batch row b, strip of PR tokens).  q and k need the norm of the
// whole H*D row: a first pass forms the per-row sums of squares (reduced
// across the workgroup through LDS), and after the barrier q and k are
// scaled by their inverse norms and stored, held in registers across the
// barrier (70 VGPRs at PR = 2; at 4 rows recomputing them after the barrier
// was 15% slower than holding them).
template <typename ST, typename GT>
__global__ __launch_bounds__(512) void producer_fwd_kernel(const ProdArgs a) {
    __shared__ float red[2][MAXW][PR];
    const Lanes L(a.H, a.D);
    const int T = a.T;
    const int nstrip = (T + PR - 1) / PR;
    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int b = wg / nstrip, t0 = (wg % nstrip) * PR;
    const size_t rb = (size_t)b * T;

    auto row_norms = [&](const float (&sv)[PR][4], int i) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < PR; ++j) {
            float ss = 0.f;
            if (L.live)
#pragma unroll
                for (int e = 0; e < 4; ++e) ss = fmaf(sv[j][e], sv[j][e], ss);
            ss = wave_sum(ss);
            if (L.lane == 0) red[i][L.w][j] = ss;
        }
    };
    float sq[PR][4], sk[PR][4];
    conv_silu_rows<ST, 0>(a, L, t0, rb, sq);
    row_norms(sq, 0);
    conv_silu_rows<ST, 1>(a, L, t0, rb, sk);
    row_norms(sk, 1);
    {
        float sv[PR][4];
        conv_silu_rows<ST, 2>(a, L, t0, rb, sv);
#pragma unroll
        for (int j = 0; j < PR; ++j)
            if (t0 + j < T && L.live) Vec4<ST>::st(static_cast<ST*>(a.v) + (rb + t0 + j) * L.HD + L.cc, sv[j]);
    }

    // decay gate, in fp32 before the cast to g's dtype (nope_gdn_mlx.py:816-820);
    // absent for the scalar-alpha layer (g == nullptr)
    if (a.g) {
        const ST* xf = static_cast<const ST*>(a.xf);
        const float4 dtv = *reinterpret_cast<const float4*>(a.dt_bias + L.cc);
        const float dt[4] = {dtv.x, dtv.y, dtv.z, dtv.w};
        const float eA = __expf(a.A_log[L.h]);
        float z[PR][4];
#pragma unroll
        for (int j = 0; j < PR; ++j) Vec4<ST>::ld(xf + (rb + min(t0 + j, T - 1)) * a.ld_f + L.cc, z[j]);
#pragma unroll
        for (int j = 0; j < PR; ++j) {
            float gv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[e] = -eA * softplus(z[j][e] + dt[e]);
            if (t0 + j < T && L.live) Vec4<GT>::st(static_cast<GT*>(a.g) + (rb + t0 + j) * L.HD + L.cc, gv);
        }
    }
    // write gate, one lane per head
    if (L.live && L.cc % a.D == 0) {
        const ST* xb = static_cast<const ST*>(a.xb);
        ST* beta = static_cast<ST*>(a.beta);
        float xv[PR];   // all loads first: one round trip, not PR
#pragma unroll
        for (int j = 0; j < PR; ++j) xv[j] = ld1<ST>(xb + (rb + min(t0 + j, T - 1)) * a.ld_b + L.h);
#pragma unroll
        for (int j = 0; j < PR; ++j)
            if (t0 + j < T) st1<ST>(beta + (rb + t0 + j) * a.H + L.h, sigm(xv[j]) * a.beta_mult);
    }

    __syncthreads();
    auto finish = [&](const float (&sv)[PR][4], int i, ST* out, float mult) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < PR; ++j) {
            float tot = 0.f;
            for (int u = 0; u < L.NW; ++u) tot += red[i][u][j];
            const float inv = mult / fmaxf(sqrtf(tot), L2_EPS);
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = sv[j][e] * inv;
            if (t0 + j < T && L.live) Vec4<ST>::st(out + (rb + t0 + j) * L.HD + L.cc, o);
        }
    };
    finish(sq, 0, static_cast<ST*>(a.q), a.scale);
    finish(sk, 1, static_cast<ST*>(a.k), 1.f);
}

// ---------------------------------------------------------------- producer, backward
// dy (the adjoint of the conv output) of tensor i for NRW rows from t0; the
// x rows t0-3 .. t0+NRW-1 come back in xr for the tap gradients.  For q and k
// the row norms reduce across the workgroup through red (one barrier).
template <typename ST, int NRW, int I>
__device__ __forceinline__ void prod_dy_rows(const ProdArgs& a, const Lanes& L, int t0, size_t rb,
                                             const float (&wt)[4][KC], const float (&bias)[4],
                                             float (*red)[2][BR], float (&dy)[NRW][4],
                                             float (&xr)[NRW + KC - 1][4]) {
    const int T = a.T;
    constexpr int i = I;
    const ST* x = static_cast<const ST*>(I == 0 ? a.xq : I == 1 ? a.xk : a.xv);
    const ST* d = static_cast<const ST*>(I == 0 ? a.dq : I == 1 ? a.dk : a.dv);
#pragma unroll
    for (int r = 0; r < NRW + KC - 1; ++r) {
        const int t = t0 - (KC - 1) + r;
        Vec4<ST>::ld(x + (rb + min(max(t, 0), T - 1)) * a.ld_x + L.cc, xr[r]);
        if (t < 0) xr[r][0] = xr[r][1] = xr[r][2] = xr[r][3] = 0.f;
    }
    float dd[NRW][4];
#pragma unroll
    for (int j = 0; j < NRW; ++j) {
        Vec4<ST>::ld(d + (rb + min(t0 + j, T - 1)) * L.HD + L.cc, dd[j]);
        if (t0 + j >= T || !L.live) dd[j][0] = dd[j][1] = dd[j][2] = dd[j][3] = 0.f;
    }
    float y[NRW][4], sg[NRW][4];
#pragma unroll
    for (int j = 0; j < NRW; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v = bias[e];
#pragma unroll
            for (int k = 0; k < KC; ++k) v = fmaf(wt[e][k], xr[j + k][e], v);
            y[j][e] = v;
            sg[j][e] = sigm(v);
        }
    float ds[NRW][4];
    if (i < 2) {
#pragma unroll
        for (int j = 0; j < NRW; ++j) {
            float ss = 0.f, dot = 0.f;
            if (L.live)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float sv = y[j][e] * sg[j][e];
                    ss = fmaf(sv, sv, ss);
                    dot = fmaf(sv, dd[j][e], dot);
                }
            ss = wave_sum(ss);
            dot = wave_sum(dot);
            if (L.lane == 0) { red[L.w][0][j] = ss; red[L.w][1][j] = dot; }
        }
        __syncthreads();
        const float mult = i == 0 ? a.scale : 1.f;
#pragma unroll
        for (int j = 0; j < NRW; ++j) {
            float ss = 0.f, dot = 0.f;
            for (int u = 0; u < L.NW; ++u) { ss += red[u][0][j]; dot += red[u][1][j]; }
            const float n = sqrtf(ss);
            // d(s / max(n, eps)) = ds / n - s (s . ds) / n^3 while n > eps, ds / eps below
            const float inv = n > L2_EPS ? 1.f / n : 1.f / L2_EPS;
            const float corr = n > L2_EPS ? dot * inv * inv : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) ds[j][e] = mult * inv * (dd[j][e] - y[j][e] * sg[j][e] * corr);
        }
    } else {
#pragma unroll
        for (int j = 0; j < NRW; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) ds[j][e] = dd[j][e];
    }
#pragma unroll
    for (int j = 0; j < NRW; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            dy[j][e] = (t0 + j < T && L.live)
                           ? ds[j][e] * sg[j][e] * (1.f + y[j][e] * (1.f - sg[j][e]))
                           : 0.f;
}

// One conv input's backward over a segment [tlo, thi) of batch row rb / T.
template <typename ST, int I>
__device__ __forceinline__ void prod_bwd_conv(const ProdArgs& a, const Lanes& L, int tlo, int thi, size_t rb,
                                              float (*red)[MAXW][2][BR], float* part) {
    constexpr int i = I;
    const int T = a.T;
    const int nst = (thi - tlo + BR - 1) / BR;
    int par = 0;
        float wt[4][KC], bias[4];
        load_taps<I>(a, L, wt, bias);
        ST* dx = static_cast<ST*>(I == 0 ? a.dxq : I == 1 ? a.dxk : a.dxv);
        float acc[KC + 1][4];
#pragma unroll
        for (int k = 0; k <= KC; ++k) acc[k][0] = acc[k][1] = acc[k][2] = acc[k][3] = 0.f;
        float carry[KC - 1][4];
        if (thi < T) {
            float xh[2 * (KC - 1)][4];
            prod_dy_rows<ST, KC - 1, I>(a, L, thi, rb, wt, bias, red[par], carry, xh);
            par ^= 1;
        } else {
#pragma unroll
            for (int r = 0; r < KC - 1; ++r) carry[r][0] = carry[r][1] = carry[r][2] = carry[r][3] = 0.f;
        }
        for (int si = nst - 1; si >= 0; --si) {
            const int t0 = tlo + si * BR;
            float dy[BR][4], xr[BR + KC - 1][4];
            prod_dy_rows<ST, BR, I>(a, L, t0, rb, wt, bias, red[par], dy, xr);
            par ^= 1;
#pragma unroll
            for (int j = 0; j < BR; ++j) {
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = 0.f;
#pragma unroll
                    for (int k = 0; k < KC; ++k) {
                        const int u = j + KC - 1 - k;   // x[t] feeds y[t + 3 - k] through tap k
                        v = fmaf(wt[e][k], u < BR ? dy[u][e] : carry[u - BR][e], v);
                    }
                    o[e] = v;
                }
                if (t0 + j < T && L.live) Vec4<ST>::st(dx + (rb + t0 + j) * a.ld_dx + L.cc, o);
            }
#pragma unroll
            for (int j = 0; j < BR; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
#pragma unroll
                    for (int k = 0; k < KC; ++k) acc[k][e] = fmaf(dy[j][e], xr[j + k][e], acc[k][e]);
                    acc[KC][e] += dy[j][e];
                }
#pragma unroll
            for (int r = 0; r < KC - 1; ++r)
#pragma unroll
                for (int e = 0; e < 4; ++e) carry[r][e] = dy[r][e];
        }
        if (L.live)
#pragma unroll
            for (int k = 0; k <= KC; ++k) Vec4<float>::st(part + (size_t)(5 * i + k) * L.HD, acc[k]);
    }

// Workgroup = (batch row b, segment of BR*BNS tokens) x role: blockIdx.y 0-2
// takes conv input q, k or v, 3 the decay and write gates, so four
// independent workgroups share a segment.  A conv input runs its strips from
// the last to the first so that the dy rows a strip needs beyond its end are
// the previous strip's (carried in registers); the three rows past the
// segment are recomputed once.  Partial sums of the parameter gradients go to
// part[wg][NPV][H*D]:
//   v = 5 i + k  tap k of conv i     v = 5 i + 4  bias of conv i
//   v = 15       dt_bias             v = 16       dg * g (summed per head -> dA_log)
template <typename ST, typename GT>
__global__ __launch_bounds__(512) void producer_bwd_kernel(const ProdArgs a) {
    __shared__ float red[2][MAXW][2][BR];
    const Lanes L(a.H, a.D);
    const int T = a.T;
    constexpr int SEG = BR * BNS;
    const int nseg = (T + SEG - 1) / SEG;
    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int b = wg / nseg, tlo = (wg % nseg) * SEG;
    const int thi = min(tlo + SEG, T);
    const size_t rb = (size_t)b * T;
    float* part = a.part + (size_t)wg * NPV * L.HD + L.cc;

    const int role = blockIdx.y;
    if (role == 0) prod_bwd_conv<ST, 0>(a, L, tlo, thi, rb, red, part);
    else if (role == 1) prod_bwd_conv<ST, 1>(a, L, tlo, thi, rb, red, part);
    else if (role == 2) prod_bwd_conv<ST, 2>(a, L, tlo, thi, rb, red, part);
    // decay gate (when present) and write gate over rows [tlo, thi)
    else {
        if (a.dg) {
            const ST* xf = static_cast<const ST*>(a.xf);
            const GT* dg = static_cast<const GT*>(a.dg);
            ST* dxf = static_cast<ST*>(a.dxf);
            const float4 dtv = *reinterpret_cast<const float4*>(a.dt_bias + L.cc);
            const float dt[4] = {dtv.x, dtv.y, dtv.z, dtv.w};
            const float eA = __expf(a.A_log[L.h]);
            float adt[4] = {0.f, 0.f, 0.f, 0.f}, aA[4] = {0.f, 0.f, 0.f, 0.f};
            for (int t0 = tlo; t0 < thi; t0 += BR) {
                float z[BR][4], dgv[BR][4];
    #pragma unroll
                for (int j = 0; j < BR; ++j) {
                    const size_t r = rb + min(t0 + j, T - 1);
                    Vec4<ST>::ld(xf + r * a.ld_f + L.cc, z[j]);
                    Vec4<GT>::ld(dg + r * L.HD + L.cc, dgv[j]);
                }
    #pragma unroll
                for (int j = 0; j < BR; ++j) {
                    const bool ok = t0 + j < thi && L.live;
                    float o[4];
    #pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float zz = z[j][e] + dt[e];
                        const float gd = ok ? dgv[j][e] : 0.f;
                        o[e] = -gd * eA * sigm(zz);
                        adt[e] += o[e];
                        aA[e] = fmaf(gd, -eA * softplus(zz), aA[e]);
                    }
                    if (ok) Vec4<ST>::st(dxf + (rb + t0 + j) * a.ld_df + L.cc, o);
                }
            }
            if (L.live) {
                Vec4<float>::st(part + (size_t)15 * L.HD, adt);
                Vec4<float>::st(part + (size_t)16 * L.HD, aA);
            }
        } else if (L.live) {   // scalar-alpha layer: no decay-gate gradients
            const float zero[4] = {0.f, 0.f, 0.f, 0.f};
            Vec4<float>::st(part + (size_t)15 * L.HD, zero);
            Vec4<float>::st(part + (size_t)16 * L.HD, zero);
        }
        if (L.live && L.cc % a.D == 0) {
            const ST* xb = static_cast<const ST*>(a.xb);
            const ST* dbeta = static_cast<const ST*>(a.dbeta);
            ST* dxb = static_cast<ST*>(a.dxb);
            for (int t0 = tlo; t0 < thi; t0 += BR) {
                float xv[BR], dv[BR];   // all loads of the strip first
#pragma unroll
                for (int j = 0; j < BR; ++j) {
                    const size_t r = rb + min(t0 + j, T - 1);
                    xv[j] = ld1<ST>(xb + r * a.ld_b + L.h);
                    dv[j] = ld1<ST>(dbeta + r * a.H + L.h);
                }
#pragma unroll
                for (int j = 0; j < BR; ++j) {
                    const float sb = sigm(xv[j]);
                    if (t0 + j < thi)
                        st1<ST>(dxb + (rb + t0 + j) * a.ld_db + L.h, dv[j] * a.beta_mult * sb * (1.f - sb));
                }
            }
        }
    }
}

// out[col] = sum_p part[p][col]; 64 columns x 4 row slices per workgroup.
// Column sums of a row-major (P, N) partial-sum buffer in a fixed order:
// workgroup (x, y) sums rows [P*y/S, P*(y+1)/S) of columns [64x, 64x + 64)
// into row y of dst, S = gridDim.y.  Four accumulators per lane keep four
// loads in flight.
__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ part, int P, int N,
                                                     float* __restrict__ dst) {
    __shared__ float red[4][64];
    const int l = threadIdx.x & 63, sl = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + l;
    const int S = gridDim.y, y = blockIdx.y;
    const int lo = (int)((long long)P * y / S), hi = (int)((long long)P * (y + 1) / S);
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    if (col < N) {
        const float* c = part + col;
        int p = lo + sl;
        for (; p + 12 < hi; p += 16) {
            s0 += c[(size_t)p * N];
            s1 += c[(size_t)(p + 4) * N];
            s2 += c[(size_t)(p + 8) * N];
            s3 += c[(size_t)(p + 12) * N];
        }
        for (; p < hi; p += 4) s0 += c[(size_t)p * N];
    }
    red[sl][l] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (sl == 0 && col < N) dst[(size_t)y * N + col] = (red[0][l] + red[1][l]) + (red[2][l] + red[3][l]);
}

__global__ __launch_bounds__(256) void producer_finish_kernel(const ProdArgs a) {
    const int HD = a.H * a.D;
    const float* cs = a.colsum;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c < HD) {
        for (int i = 0; i < 3; ++i) {
#pragma unroll
            for (int k = 0; k < KC; ++k) a.dconv_w[((size_t)i * HD + c) * KC + k] = cs[(size_t)(5 * i + k) * HD + c];
            if (a.dconv_b) a.dconv_b[(size_t)i * HD + c] = cs[(size_t)(5 * i + KC) * HD + c];
        }
        if (a.ddt_bias) a.ddt_bias[c] = cs[(size_t)15 * HD + c];
    }
    // dA_log[h] = sum over the head's D channels: one wave per head, the
    // lanes over channels (the loop bound is the same for the whole wave)
    if (a.dA_log) {
        const int lane = threadIdx.x & 63;
        for (int h = blockIdx.x * 4 + (threadIdx.x >> 6); h < a.H; h += gridDim.x * 4) {
            float s = 0.f;
            for (int d = lane; d < a.D; d += 64) s += cs[(size_t)16 * HD + (size_t)h * a.D + d];
            s = wave_sum(s);
            if (lane == 0) a.dA_log[h] = s;
        }
    }
}

// ---------------------------------------------------------------- gated RMSNorm
// Lanes of the norm kernels: a head takes P lanes of 4 channels, P = D / 4
// rounded up to a power of two, so that its sums are butterflies over an
// aligned lane group; a wave holds 64 / P heads.  For D a power of two this is
// the channel-contiguous map of Lanes (256 channels a wave).  Lanes past a
// head's D / 4 (D = 96: 8 of 32) are idle: they address channel 0 and add
// zero to the sums.
__device__ __forceinline__ int norm_lanes_per_head(int D) {
    int p = 1;
    while (4 * p < D) p <<= 1;
    return p;
}
struct NormLanes {
    int HD, cc, P;
    bool live;
    __device__ NormLanes(int H, int D) {
        HD = H * D;
        P = norm_lanes_per_head(D);
        const int lane = threadIdx.x & 63, h = (threadIdx.x >> 6) * (64 / P) + lane / P, c4 = (lane % P) * 4;
        live = h < H && c4 < D;
        cc = live ? h * D + c4 : 0;
    }
};

template <typename ST>
__global__ __launch_bounds__(512) void rmsnorm_fwd_kernel(const NormArgs a) {
    const NormLanes L(a.H, a.D);
    const int r0 = xcd_remap(blockIdx.x, gridDim.x) * NR;
    const int gl = L.P;
    const float4 wv = *reinterpret_cast<const float4*>(a.w + L.cc % a.D);
    const float wt[4] = {wv.x, wv.y, wv.z, wv.w};
    const float invD = 1.f / (float)a.D;
    const ST* o = static_cast<const ST*>(a.o);
    const ST* z = static_cast<const ST*>(a.z);
    float ov[NR][4], zv[NR][4];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const size_t r = min(r0 + j, a.rows - 1);
        Vec4<ST>::ld(o + r * L.HD + L.cc, ov[j]);
        Vec4<ST>::ld(z + r * a.ld_z + L.cc, zv[j]);
        if (!L.live) ov[j][0] = ov[j][1] = ov[j][2] = ov[j][3] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = fmaf(ov[j][e], ov[j][e], ss);
        ss = lanes_sum(ss, gl);
        const float rs = rsqrtf(ss * invD + a.eps);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = ov[j][e] * rs * wt[e] * sigm(zv[j][e]);
        if (r0 + j < a.rows && L.live) Vec4<ST>::st(static_cast<ST*>(a.y) + (size_t)(r0 + j) * a.ld_y + L.cc, y);
    }
}

// n = o r, r = (mean(o^2) + eps)^-1/2, y = n w s(z):
//   dn = dy w s,  do = r (dn - n mean(dn n)),  dz = dy n w s (1 - s),  dw += dy n s
template <typename ST>
__global__ __launch_bounds__(512) void rmsnorm_bwd_kernel(const NormArgs a) {
    const NormLanes L(a.H, a.D);
    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int gl = L.P;
    const float4 wv = *reinterpret_cast<const float4*>(a.w + L.cc % a.D);
    const float wt[4] = {wv.x, wv.y, wv.z, wv.w};
    const float invD = 1.f / (float)a.D;
    const ST* o = static_cast<const ST*>(a.o);
    const ST* z = static_cast<const ST*>(a.z);
    const ST* dyp = static_cast<const ST*>(a.dy);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < NNS; ++s) {
        const int r0 = (wg * NNS + s) * NRB;
        if (r0 >= a.rows) break;
        float ov[NRB][4], zv[NRB][4], gv[NRB][4];
#pragma unroll
        for (int j = 0; j < NRB; ++j) {
            const size_t r = min(r0 + j, a.rows - 1);
            Vec4<ST>::ld(o + r * L.HD + L.cc, ov[j]);
            Vec4<ST>::ld(z + r * a.ld_z + L.cc, zv[j]);
            Vec4<ST>::ld(dyp + r * a.ld_dy + L.cc, gv[j]);
            if (!L.live) ov[j][0] = ov[j][1] = ov[j][2] = ov[j][3] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < NRB; ++j) {
            const bool ok = r0 + j < a.rows && L.live;
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) ss = fmaf(ov[j][e], ov[j][e], ss);
            ss = lanes_sum(ss, gl);
            const float rs = rsqrtf(ss * invD + a.eps);
            float n[4], sg[4], dn[4], dot = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                n[e] = ov[j][e] * rs;
                sg[e] = sigm(zv[j][e]);
                dn[e] = gv[j][e] * wt[e] * sg[e];
                dot = fmaf(dn[e], n[e], dot);
            }
            dot = lanes_sum(dot, gl) * invD;
            float od[4], zd[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                od[e] = rs * (dn[e] - n[e] * dot);
                zd[e] = dn[e] * n[e] * (1.f - sg[e]);
                if (ok) acc[e] = fmaf(gv[j][e] * n[e], sg[e], acc[e]);
            }
            if (ok) {
                const size_t r = r0 + j;
                Vec4<ST>::st(static_cast<ST*>(a.dout) + r * L.HD + L.cc, od);
                Vec4<ST>::st(static_cast<ST*>(a.dz) + r * a.ld_dz + L.cc, zd);
            }
        }
    }
    if (L.live) Vec4<float>::st(a.part + (size_t)wg * L.HD + L.cc, acc);
}

__global__ __launch_bounds__(256) void rmsnorm_finish_kernel(const NormArgs a) {
    const int d = threadIdx.x;
    if (d < a.D) {
        float s = 0.f;
        for (int h = 0; h < a.H; ++h) s += a.colsum[(size_t)h * a.D + d];
        a.dw[d] = s;
    }
}

int nwaves(int H, int D) { return (H * D + CPW - 1) / CPW; }

// Row slices of the first column-sum pass: about 1024 workgroups over the
// chip, at least 8 rows a slice, at most 64 slices (the second pass sums them).
int colsum_splits(int P, int N) {
    const int nbx = (N + 63) / 64;
    return std::max(1, std::min({(1024 + nbx - 1) / nbx, P / 8, 64}));
}

// Column sums of part (P, N) into out (N), through stage (colsum_splits rows
// of N) when the rows are split.
void launch_colsum(const float* part, int P, int N, float* out, float* stage, hipStream_t st) {
    const int nbx = (N + 63) / 64, S = colsum_splits(P, N);
    if (S == 1) {
        colsum_kernel<<<dim3(nbx, 1), dim3(256), 0, st>>>(part, P, N, out);
        return;
    }
    colsum_kernel<<<dim3(nbx, S), dim3(256), 0, st>>>(part, P, N, stage);
    colsum_kernel<<<dim3(nbx, 1), dim3(256), 0, st>>>(stage, S, N, out);
}

}  // namespace

// waves of the norm kernels (NormLanes): 64 / P heads a wave
int norm_waves(int H, int D) {
    int p = 1;
    while (4 * p < D) p <<= 1;
    const int hpw = 64 / p;
    return (H + hpw - 1) / hpw;
}

int producer_partials(int B, int T) { return B * ((T + BR * BNS - 1) / (BR * BNS)); }
size_t producer_ws_floats(int B, int T, int H, int D) {
    const int P = producer_partials(B, T), N = NPV * H * D;
    return ((size_t)P + 1 + colsum_splits(P, N)) * N;
}
int rmsnorm_partials(int rows) { return (rows + NRB * NNS - 1) / (NRB * NNS); }
size_t rmsnorm_ws_floats(int rows, int H, int D) {
    const int P = rmsnorm_partials(rows), N = H * D;
    return ((size_t)P + 1 + colsum_splits(P, N)) * N;
}

hipError_t launch_producer_fwd(const ProdArgs& a, int in_bf16, int g_bf16, hipStream_t st) {
    const dim3 grid(a.B * ((a.T + PR - 1) / PR)), block(64 * nwaves(a.H, a.D));
    if (in_bf16) {
        if (g_bf16) producer_fwd_kernel<uint16_t, uint16_t><<<grid, block, 0, st>>>(a);
        else producer_fwd_kernel<uint16_t, float><<<grid, block, 0, st>>>(a);
    } else {
        if (g_bf16) producer_fwd_kernel<float, uint16_t><<<grid, block, 0, st>>>(a);
        else producer_fwd_kernel<float, float><<<grid, block, 0, st>>>(a);
    }
    return hipGetLastError();
}

hipError_t launch_producer_bwd(const ProdArgs& a, int in_bf16, int g_bf16, hipStream_t st) {
    const int P = producer_partials(a.B, a.T);
    const int HD = a.H * a.D;
    const dim3 grid(P, 4), block(64 * nwaves(a.H, a.D));
    if (P == 0) {
        // no rows: the column sums below still write the (zero) parameter gradients
    } else if (in_bf16) {
        if (g_bf16) producer_bwd_kernel<uint16_t, uint16_t><<<grid, block, 0, st>>>(a);
        else producer_bwd_kernel<uint16_t, float><<<grid, block, 0, st>>>(a);
    } else {
        if (g_bf16) producer_bwd_kernel<float, uint16_t><<<grid, block, 0, st>>>(a);
        else producer_bwd_kernel<float, float><<<grid, block, 0, st>>>(a);
    }
    const int N = NPV * HD;
    launch_colsum(a.part, P, N, a.colsum, a.colsum + N, st);
    producer_finish_kernel<<<dim3((HD + 255) / 256), dim3(256), 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_fwd(const NormArgs& a, int in_bf16, hipStream_t st) {
    const dim3 grid((a.rows + NR - 1) / NR), block(64 * norm_waves(a.H, a.D));
    if (in_bf16) rmsnorm_fwd_kernel<uint16_t><<<grid, block, 0, st>>>(a);
    else rmsnorm_fwd_kernel<float><<<grid, block, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_bwd(const NormArgs& a, int in_bf16, hipStream_t st) {
    const int P = rmsnorm_partials(a.rows);
    const int HD = a.H * a.D;
    const dim3 grid(P), block(64 * norm_waves(a.H, a.D));
    if (P > 0) {
        if (in_bf16) rmsnorm_bwd_kernel<uint16_t><<<grid, block, 0, st>>>(a);
        else rmsnorm_bwd_kernel<float><<<grid, block, 0, st>>>(a);
    }
    launch_colsum(a.part, P, HD, a.colsum, a.colsum + HD, st);
    rmsnorm_finish_kernel<<<dim3(1), dim3(256), 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace kda
