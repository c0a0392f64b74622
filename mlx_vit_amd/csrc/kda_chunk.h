// kda_chunk.h -- workgroup-level phases shared by the per-chunk kernels
// (forward prep and backward local adjoints).  One workgroup = 256 threads =
// 4 waves works on one (batch, head, chunk) of C = 64 tokens.
//
// Anchored decay products.  For rows t, s of one chunk with gamma the in-chunk
// cumulative log-decay, the pair weight exp(gamma_t - gamma_s) (s <= t) is split
// at the anchor r = 16 * (t / 16), the first row of t's 16-row sub-block:
//     exp(gamma_t - gamma_r) * exp(gamma_r - gamma_s).
// Off the diagonal sub-block both factors are <= 1.  On the diagonal sub-block
// the second factor is bounded by the sub-block's decay span, which the span
// guard limits to SPAN_MAX; a chunk that fails the guard (or has any g > 0)
// takes the pairwise path instead, which evaluates every exp(gamma_t - gamma_s)
// directly, as the reference's M kernel does (nope_gdn_mlx.py:1319-1334).
//
// LDS holds, per chunk (fp32, rows padded by 4 floats against bank conflicts):
//   g  : gamma                      (raw g until the cumsum)
//   kl : k_t e^{gamma_t - gamma_r}  (A operand, left factor)
//   ql : q_t e^{gamma_t - gamma_r}  (raw q until the transform)
//   kr : k_s e^{gamma_r' - gamma_s} with r' the anchor of s's own sub-block
//        (raw k until the transform); the right factor for sub-block row i is
//        kr * f[i][j], f[i][j] = e^{gamma_16i - gamma_16j}
//   er : e^{gamma_r} per sub-block and channel
#pragma once
#include "kda_device.h"

namespace kda {

template <int D>
struct ChunkLds {
    float g[C][D + 4];
    float kl[C][D + 4];
    float ql[C][D + 4];
    float kr[C][D + 4];
    union {
        struct {
            float er[NB][D];
            float f[6][D];
        };
        struct {         // pairwise path only, where f is not used; written after er / f
            float er_keep[NB][D];
            float bw[C];            // slowest-channel decay cumsum
            uint16_t bpre[C + 1];   // band-width prefix sums (< 2081)
            uint8_t blo[C], bhi[C]; // decay band of each row
        };
        float tmp[256];  // cumsum partial totals; dead before er / f are written
    };
    float beta[C];
};

// pair index of sub-block pair (i, j), j < i: (1,0)=0 (2,0)=1 (2,1)=2 (3,0)=3 (3,1)=4 (3,2)=5
__device__ __forceinline__ int pair_idx(int i, int j) { return (i * (i - 1)) / 2 + j; }

// lower sub-block tiles (i, j <= i) enumerated 0..9
__device__ __forceinline__ void tile_ij(int tix, int& i, int& j) {
    i = (tix >= 6) ? 3 : (tix >= 3) ? 2 : (tix >= 1) ? 1 : 0;
    j = tix - (i * (i + 1)) / 2;
}

template <int PREC> __device__ __forceinline__ float kexp(float x) {
    if constexpr (PREC == 1) return __expf(x);
    else return expf(x);
}

// Load one chunk of q, k, g, beta (rows >= valid are zero: g = 0 no decay,
// beta = 0 no write -- the reference's padding, nope_gdn_mlx.py:2354-2361).
// Returns 1 if this thread saw g > 0 (or a NaN), which disables the anchored path.
template <int D, typename TI, typename TG>
__device__ int chunk_load(ChunkLds<D>& s, const TI* __restrict__ q, const TI* __restrict__ k,
                          const TG* __restrict__ g, const TI* __restrict__ beta, size_t base,
                          size_t rstride, size_t bbase, int H, int valid) {
    const int tid = threadIdx.x;
    int flag = 0;
    constexpr int Q4 = D / 4;
    for (int idx = tid; idx < C * Q4; idx += 256) {
        const int t = idx / Q4, d = (idx % Q4) * 4;
        float4 vq = make_float4(0.f, 0.f, 0.f, 0.f), vk = vq, vg = vq;
        if (t < valid) {
            const size_t o = base + (size_t)t * rstride + d;
            vq = ld4<TI>(q + o);
            vk = ld4<TI>(k + o);
            vg = ld4<TG>(g + o);
        }
        *reinterpret_cast<float4*>(&s.ql[t][d]) = vq;
        *reinterpret_cast<float4*>(&s.kr[t][d]) = vk;
        *reinterpret_cast<float4*>(&s.g[t][d]) = vg;
        if (!(vg.x <= 0.f && vg.y <= 0.f && vg.z <= 0.f && vg.w <= 0.f)) flag = 1;
    }
    if (tid < C) s.beta[tid] = (tid < valid) ? ld1<TI>(beta + bbase + (size_t)tid * H) : 0.f;
    __syncthreads();
    return flag;
}

// In-place inclusive cumsum of s.g over rows, per channel.
template <int D>
__device__ void chunk_cumsum(ChunkLds<D>& s) {
    constexpr int PARTS = 256 / D, RP = C / PARTS;
    const int tid = threadIdx.x, d = tid % D, p = tid / D;
    float run = 0.f;
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        run += s.g[p * RP + r][d];
        s.g[p * RP + r][d] = run;
    }
    s.tmp[p * D + d] = run;
    __syncthreads();
    float off = 0.f;
    for (int pp = 0; pp < p; ++pp) off += s.tmp[pp * D + d];
    if (p > 0) {
#pragma unroll
        for (int r = 0; r < RP; ++r) s.g[p * RP + r][d] += off;
    }
    __syncthreads();
}

// Anchor factors er, f and the span guard.  Returns nonzero (uniform over the
// workgroup) when the chunk must take the pairwise path.
template <int D, int PREC>
__device__ int chunk_factors(ChunkLds<D>& s, int flag) {
    const int tid = threadIdx.x;
    for (int idx = tid; idx < NB * D; idx += 256) {
        const int j = idx / D, d = idx % D;
        const float span = s.g[BS * j][d] - s.g[BS * j + BS - 1][d];
        if (!(span <= SPAN_MAX)) flag = 1;
        s.er[j][d] = kexp<PREC>(s.g[BS * j][d]);
    }
    for (int idx = tid; idx < 6 * D; idx += 256) {
        const int p = idx / D, d = idx % D;
        const int i = (p >= 3) ? 3 : (p >= 1) ? 2 : 1;
        const int j = p - pair_idx(i, 0);
        s.f[p][d] = kexp<PREC>(s.g[BS * i][d] - s.g[BS * j][d]);
    }
    return __syncthreads_or(flag);
}

// kl = k e^{g_t - g_r}, ql = q e^{g_t - g_r}; with `anchored`, kr = k e^{g_r - g_t}
// (otherwise kr keeps raw k).  Raw q, k are read from ql, kr.  The caller
// syncs afterwards.
template <int D, int PREC>
__device__ void chunk_transform(ChunkLds<D>& s, bool anchored) {
    const int tid = threadIdx.x;
    for (int idx = tid; idx < C * D; idx += 256) {
        const int t = idx / D, d = idx % D, r = t & ~(BS - 1);
        const float x = s.g[t][d] - s.g[r][d];
        const float el = kexp<PREC>(x);
        const float kv = s.kr[t][d], qv = s.ql[t][d];
        s.kl[t][d] = kv * el;
        s.ql[t][d] = qv * el;
        if (anchored) s.kr[t][d] = kv * kexp<PREC>(-x);
    }
}

// Unit-lower inverses of the four 16x16 diagonal blocks of (I + L), by forward
// substitution in fp32: wave w inverts block w, lane c (< 16) owns column c.
// L is read from a row-major LDS matrix (leading dimension ldl); the inverse
// goes to tii[w][row][col].
template <int LDL>
__device__ void diag_inverse(const float* __restrict__ L, float (*tii)[BS][BS + 4], int nblocks) {
    const int w = threadIdx.x >> 6, c = threadIdx.x & 63;
    if (w < nblocks && c < BS) {
        const float* Lb = L + (size_t)(BS * w) * LDL + BS * w;
        float x[BS];
#pragma unroll
        for (int t = 0; t < BS; ++t) {
            float acc = (t == c) ? 1.f : 0.f;
#pragma unroll
            for (int j = 0; j < t; ++j) acc -= Lb[t * LDL + j] * x[j];
            x[t] = acc;
        }
#pragma unroll
        for (int t = 0; t < BS; ++t) tii[w][t][c] = x[t];
    }
}

}  // namespace kda

// ============================================================================
// Typed-storage chunk phases (ST = bf16 for bf16 inputs, fp32 otherwise).
// q, k, v and the anchored operands are kept in ST; gamma and the small
// factor tables in fp32.  Rows are padded by 16 bytes.
// ============================================================================
namespace kda {

template <int D, typename ST>
struct ChunkSmem {
    // fp32 storage at D = 128 drops the row pad to fit in 160 KB
    static constexpr bool TIGHT = sizeof(ST) == 4 && D >= 128;
    static constexpr int PS = TIGHT ? 0 : 16 / (int)sizeof(ST);
    static constexpr int LDK = D + PS;     // ST rows
    static constexpr int LDG = D + (TIGHT ? 0 : 4);   // fp32 rows
    ST kl[C][LDK];     // k e^{g_t - g_r}
    ST ql[C][LDK];     // raw q, then q e^{g_t - g_r}
    ST kr[C][LDK];     // raw k, then k e^{g_r - g_t} (anchored path)
    float g[C][LDG];   // raw g, then gamma
    union {
        struct {
            float er[NB][D];    // e^{gamma_16j}
            float egr[NB][D];   // e^{G - gamma_16j}
            float f[6][D];      // e^{gamma_16i - gamma_16j}, j < i
        };
        struct {                // pairwise path only, where egr and f are not used;
            float er_keep[NB][D];   // written after the factor tables
            float bw[C];            // slowest-channel decay cumsum
            uint16_t bpre[C + 1];   // band-width prefix sums (< 2081)
            uint8_t blo[C], bhi[C]; // decay band of each row
        };
        float tmp[512];
    };
    float beta[C];
};

// All 16-byte loads of one chunk of q, k, g, beta (and optionally v) are issued
// before anything is written to LDS; every wave's q, k, g, beta requests enter
// the memory pipeline before any v request.  v stays in tv for the caller to
// store once its latency is hidden.  Rows >= valid are zero.  Returns 1 if this
// thread saw g > 0 or a NaN.
template <int D, typename ST, typename TG, bool WITH_V>
__device__ __forceinline__ int chunk_load2(ChunkSmem<D, ST>& s, Tile<ST, C, D>& tv, const ST* __restrict__ q,
                                           const ST* __restrict__ k, const ST* __restrict__ v,
                                           const TG* __restrict__ g, const ST* __restrict__ beta, size_t base,
                                           size_t rstride, size_t bbase, int H, int valid) {
    Tile<ST, C, D> tq, tk;
    Tile<TG, C, D> tg;
    tq.load(q + base, rstride, valid);
    tk.load(k + base, rstride, valid);
    tg.load(g + base, rstride, valid);
    const int tid = threadIdx.x;
    const float braw = ld1<ST>(beta + bbase + (size_t)min(tid, valid - 1) * H);
    if constexpr (WITH_V) {
        __builtin_amdgcn_s_barrier();
        tv.load(v + base, rstride, valid);
    }
    tq.store(&s.ql[0][0], ChunkSmem<D, ST>::LDK);
    tk.store(&s.kr[0][0], ChunkSmem<D, ST>::LDK);
    int flag = 0;
    constexpr int EPV = Tile<TG, C, D>::EPV, VPR = Tile<TG, C, D>::VPR;
#pragma unroll
    for (int i = 0; i < Tile<TG, C, D>::PER; ++i) {
        const int vv = tid + 256 * i;
        const int row = vv / VPR, c = (vv - row * VPR) * EPV;
        const Vec16<TG> x{tg.get(i)};
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
            const float gv = x.get(e);
            s.g[row][c + e] = gv;
            if (!(gv <= 0.f)) flag = 1;
        }
    }
    if (tid < C) s.beta[tid] = (tid < valid) ? braw : 0.f;
    __syncthreads();
    return flag;
}

template <int D, typename ST, int NTH = 256>
__device__ __forceinline__ void chunk_cumsum2(ChunkSmem<D, ST>& s) {
    constexpr int PARTS = NTH / D, RP = C / PARTS;
    static_assert(PARTS * D <= 512, "cumsum partials fit tmp");
    const int tid = threadIdx.x, d = tid % D, p = tid / D;
    float run = 0.f;
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        run += s.g[p * RP + r][d];
        s.g[p * RP + r][d] = run;
    }
    s.tmp[p * D + d] = run;
    __syncthreads();
    float off = 0.f;
    for (int pp = 0; pp < p; ++pp) off += s.tmp[pp * D + d];
    if (p > 0) {
#pragma unroll
        for (int r = 0; r < RP; ++r) s.g[p * RP + r][d] += off;
    }
    __syncthreads();
}

// factor tables + span guard; returns nonzero (uniform) for the pairwise path
template <int D, typename ST, int PREC, int NTH = 256>
__device__ __forceinline__ int chunk_factors2(ChunkSmem<D, ST>& s, int flag) {
    const int tid = threadIdx.x;
    for (int idx = tid; idx < NB * D; idx += NTH) {
        const int j = idx / D, d = idx % D;
        const float g0 = s.g[BS * j][d];
        const float span = g0 - s.g[BS * j + BS - 1][d];
        if (!(span <= SPAN_MAX)) flag = 1;
        s.er[j][d] = kexp<PREC>(g0);
        s.egr[j][d] = kexp<PREC>(s.g[C - 1][d] - g0);
    }
    for (int idx = tid; idx < 6 * D; idx += NTH) {
        const int p = idx / D, d = idx % D;
        const int i = (p >= 3) ? 3 : (p >= 1) ? 2 : 1;
        const int j = p - pair_idx(i, 0);
        s.f[p][d] = kexp<PREC>(s.g[BS * i][d] - s.g[BS * j][d]);
    }
    return __syncthreads_or(flag);
}

// Register-resident inverses of the four 16x16 diagonal blocks of I + L,
// L[t][s] = beta_t Akk[t][s]: wave w inverts block w, lane c (< 16) owns
// column c.  All 36 row reads of the block's strict lower part are issued
// before the substitution starts (one LDS round trip instead of one per row);
// beta_t scales the row sum: x_t = [t == c] - beta_t sum_{s<t} Akk[t][s] x_s.
// With fc != nullptr the block's transpose is also written as split (PREC 3)
// MFMA A fragments, fc[64 w + lane] = fragment of lane (g, r) holding
// T_ww[4g + e][r], so that other waves load it with one 16-byte read per lane.
template <int LDA>
__device__ __forceinline__ void diag_inverse_reg(const float* __restrict__ akk, const float* __restrict__ beta,
                                                 float (*tii)[BS][BS + 4], Frag4* fc = nullptr) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), c = threadIdx.x & 63;
    if (c < BS) {
        const float* Ab = akk + (size_t)(BS * w) * LDA + BS * w;
        float4 R[BS][BS / 4];
        float bt[BS];
#pragma unroll
        for (int t = 1; t < BS; ++t) {
            bt[t] = beta[BS * w + t];
#pragma unroll
            for (int j4 = 0; j4 < (t + 3) / 4; ++j4) R[t][j4] = *reinterpret_cast<const float4*>(Ab + t * LDA + 4 * j4);
        }
        __builtin_amdgcn_sched_barrier(0);
        float x[BS];
        x[0] = (c == 0) ? 1.f : 0.f;
#pragma unroll
        for (int t = 1; t < BS; ++t) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < t; ++j) {
                const float4 r = R[t][j / 4];
                const float a = (j % 4 == 0) ? r.x : (j % 4 == 1) ? r.y : (j % 4 == 2) ? r.z : r.w;
                acc += a * x[j];
            }
            x[t] = ((t == c) ? 1.f : 0.f) - bt[t] * acc;
        }
#pragma unroll
        for (int t = 0; t < BS; ++t) tii[w][t][c] = x[t];
        if (fc) {
#pragma unroll
            for (int g = 0; g < 4; ++g) fc[64 * w + 16 * g + c] = frag4_from_f32<3>(&x[4 * g]);
        }
    }
}


// Decay band of every row for the pairwise path.  With gamma non-increasing in
// t (every g <= 0), let w_u = min over channels of gamma_{u-1} - gamma_u (the
// slowest channel's decay at step u) and W its cumsum: every channel decays by
// at least W_t - W_s between rows s < t, so exp(gamma_t - gamma_s) <
// e^{-BAND_CUT} in all channels once W_t - W_s > BAND_CUT.  blo[t] / bhi[t] are
// the first / last rows s with W within BAND_CUT of W_t; pairs outside
// contribute below 1.8e-35 of an O(1) term and are skipped.  A chunk with any
// g > 0 or NaN (nonmono) keeps the full range.  Also sets bpre[t] = sum over
// u < t of (u - blo[u] + 1), bpre[C] the total.  Called by the whole
// workgroup (barriers inside); the arrays are ready after.
constexpr float BAND_CUT = 80.0f;
template <int D, int NTH, typename S>
__device__ void chunk_band(S& s, int nonmono) {
    static_assert(C == 64, "one lane per row in the scans below");
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    constexpr int NW = NTH / 64;
    if (!nonmono) {
        for (int u = w; u < C; u += NW) {
            float m = 3.0e38f;
            if (u > 0)
                for (int d = lane; d < D; d += 64) m = fminf(m, s.g[u - 1][d] - s.g[u][d]);
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) m = fminf(m, __shfl_xor(m, o));
            if (lane == 0) s.bw[u] = (u > 0) ? m : 0.f;
        }
    }
    __syncthreads();
    if (w == 0) {
        // W = inclusive scan of w over the rows; then the band by binary search
        float W = nonmono ? 0.f : s.bw[lane];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float x = __shfl_up(W, o);
            if (lane >= o) W += x;
        }
        s.bw[lane] = W;
        // one wave: its LDS writes are done before its reads below (no barrier here,
        // the other waves wait at the one after this block)
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        int lo = 0, hi = C - 1;
        if (!nonmono) {
            // first s <= t with W_s >= W_t - CUT, last s >= t with W_s <= W_t + CUT
            int a = 0, b = lane;
            while (a < b) {
                const int m = (a + b) >> 1;
                if (s.bw[m] >= W - BAND_CUT) b = m;
                else a = m + 1;
            }
            lo = a;
            a = lane;
            b = C - 1;
            while (a < b) {
                const int m = (a + b + 1) >> 1;
                if (s.bw[m] <= W + BAND_CUT) a = m;
                else b = m - 1;
            }
            hi = a;
        }
        s.blo[lane] = (uint8_t)lo;
        s.bhi[lane] = (uint8_t)hi;
        // exclusive scan of the band widths (pairs s <= t)
        const int wdt = lane - lo + 1;
        int inc = wdt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int x = __shfl_up(inc, o);
            if (lane >= o) inc += x;
        }
        s.bpre[lane] = (uint16_t)(inc - wdt);
        if (lane == C - 1) s.bpre[C] = (uint16_t)inc;
    }
    __syncthreads();
}

// Row t of the band pair with index q (0 <= q < bpre[C]): the largest t with
// bpre[t] <= q; the pair is (t, blo[t] + q - bpre[t]).
template <typename S>
__device__ __forceinline__ int band_row(const S& s, int q) {
    int lo = 0, hi = C;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s.bpre[mid] <= q) lo = mid;
        else hi = mid;
    }
    return lo;
}

}  // namespace kda
