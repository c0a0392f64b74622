// kda_chunk.h -- workgroup-level phases shared by the per-chunk kernels
// (forward prep and backward local adjoints), which work on one (batch, head,
// chunk) of C = 64 tokens per workgroup.
//
// ChunkLds and its phases serve the fp32 local-adjoint kernel; ChunkSmem (below)
// the prep and bf16 local-adjoint kernels, with block-end anchoring.
//
// Anchored decay products (ChunkLds).  For rows t, s of one chunk with gamma the in-chunk
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

// Block-end anchored decay products (the ChunkSmem kernels: prep and the bf16
// local adjoints).  Rows fall in NB blocks of BS = 16; with gamma the in-chunk
// cumulative log-decay and gamma_{-1} = 0, block i spans rows 16i .. 16i+15:
//   a_t = gamma_t - gamma_{16i-1}        in-block inclusive cumsum of g (<= 0)
//   b_t = gamma_{16i+15} - gamma_t = T_i - a_t,  T_i = a_{16i+15}  (<= 0)
// For s in block j < i, t in block i the pair weight splits into factors that
// are all <= 1, whatever the decay:
//   e^{gamma_t - gamma_s} = e^{a_t} * F_ij * e^{b_s},   F_ij = e^{T_{j+1} + ... + T_{i-1}}
// so K_l = K e^{a} and Q_l = Q e^{a} are the row operands, K_r = K e^{b} the
// column operand, and F_ij (1 for adjacent blocks) scales the product per
// channel.  On the diagonal tile (s, t in block i) the weight is
// e^{a_t} e^{-T_i} e^{b_s}: the factor e^{-T_i} >= 1 is the block's decay
// span, kept when span_i = -T_i <= SPAN_MAX; a block with a larger span has its
// diagonal tile evaluated pair by pair, e^{a_t - a_s}, and only that tile.
// Every exponent is a sum of in-block cumsums and block totals, so its fp32
// error scales with one block's span, not with the chunk's whole decay.
// A chunk with g > 0 or a NaN anywhere (outside the layer's domain, where the
// factors could exceed 1) is evaluated entirely pair by pair.
template <int D, typename ST>
struct ChunkSmem {
    // fp32 storage at D = 128 drops the row pad to fit in 160 KB
    static constexpr bool TIGHT = sizeof(ST) == 4 && D >= 128;
    static constexpr int PS = TIGHT ? 0 : 16 / (int)sizeof(ST);
    static constexpr int LDK = D + PS;     // ST rows
    static constexpr int LDG = D + (TIGHT ? 0 : 4);   // fp32 rows
    ST kl[C][LDK];     // k e^{a_t}
    ST ql[C][LDK];     // raw q, then q e^{a_t}
    ST kr[C][LDK];     // raw k, then k e^{b_t} (anchored chunks)
    float g[C][LDG];   // a (in-block inclusive cumsum of g, formed at load)
    float fac[14][D];  // factor tables, rows FAC_* below
    float beta[C];
};

// rows of ChunkSmem::fac, per channel
constexpr int FAC_EP = 0;   // + i - 1, i = 1..3: e^{gamma_{16i-1}} = e^{T_0 + .. + T_{i-1}}
constexpr int FAC_EQ = 3;   // + j, j = 0..2:     e^{G - gamma_{16j+15}} = e^{T_{j+1} + .. + T_3}
constexpr int FAC_F = 6;    // (2,0), (3,1), (3,0): F_ij for non-adjacent blocks
constexpr int FAC_FD = 9;   // + i, i = 0..3:     e^{min(-T_i, SPAN_MAX)}
constexpr int FAC_ONE = 13;  // 1: the factor of the blocks the rows above skip
// e^{gamma_{16i-1}}: e^{gamma} at the end of the block before i (1 for i = 0)
template <int D, typename ST>
__device__ __forceinline__ float fac_ep(const ChunkSmem<D, ST>& s, int i, int d) {
    return i == 0 ? 1.f : s.fac[FAC_EP + i - 1][d];
}
// e^{G - gamma_{16j+15}}: the decay from the end of block j to the chunk end (1 for j = 3)
template <int D, typename ST>
__device__ __forceinline__ float fac_eq(const ChunkSmem<D, ST>& s, int j, int d) {
    return j == NB - 1 ? 1.f : s.fac[FAC_EQ + j][d];
}
// row of F_ij, j < i - 1 (adjacent blocks have F = 1 and no row)
__device__ __forceinline__ int fac_f_row(int i, int j) { return FAC_F + ((i == 2) ? 0 : (j == 1) ? 1 : 2); }
// the per-channel factor of tile (i, j), j <= i: F_ij, or e^{-T_i} on the diagonal
template <int D, typename ST>
__device__ __forceinline__ float fac_tile(const ChunkSmem<D, ST>& s, int i, int j, int d) {
    return (j == i) ? s.fac[FAC_FD + i][d] : (j == i - 1) ? 1.f : s.fac[fac_f_row(i, j)][d];
}

// All 16-byte loads of one chunk of q, k, g, beta (and optionally v) are issued
// before anything is written to LDS; every wave's q, k, g, beta requests enter
// the memory pipeline before any v request.  v stays in tv for the caller to
// store once its latency is hidden.  Rows >= valid are zero.  g is loaded as
// lane (row 16 b + r16 of block b, 8-channel groups): the 16 rows of a block
// sit in the 16 lanes of one DPP row, so s.g receives a, the inclusive cumsum
// of g inside each 16-row block, computed by a four-step lane scan.  NTH
// threads: NTH / 256 waves per block, wave w covering block w / (NTH / 256)
// and the channel groups 4 (w % (NTH / 256)) + g4 + 4 (NTH / 256) cp.
// Returns 1 if this thread saw g > 0 or a NaN.
template <int D, typename ST, typename TG, bool WITH_V, int NTH = 256>
__device__ __forceinline__ int chunk_load2(ChunkSmem<D, ST>& s, Tile<ST, C, D, NTH>& tv, const ST* __restrict__ q,
                                           const ST* __restrict__ k, const ST* __restrict__ v,
                                           const TG* __restrict__ g, const ST* __restrict__ beta, size_t base,
                                           size_t rstride, size_t bbase, int H, int valid, int dio = D) {
    // GH: one decay per (b, t, h) (TG = GHead), read once per row and shared by
    // the lane's channels
    constexpr bool GH = std::is_same<TG, GHead>::value;
    using TGE = typename std::conditional<GH, float, TG>::type;
    constexpr int WPB = NTH / 256, NCG = D / 8, CPL = NCG / (4 * WPB), GV = GH ? 1 : 8 * (int)sizeof(TGE) / 16,
                  GE = 16 / (int)sizeof(TGE);
    static_assert(NB == 4 && NCG % (4 * WPB) == 0, "whole 8-channel groups per lane");
    // NARROW: the tensors' rows hold dio < D channels (a multiple of 8); the
    // tile's channels past dio read as zero
    constexpr bool NARROW_OK = D == 128;
    const bool narrow = NARROW_OK && dio < D;
    Tile<ST, C, D, NTH> tq, tk;
    const int tid = threadIdx.x, w = tid >> 6, r16 = tid & 15, g4 = (tid >> 4) & 3;
    const int grow = BS * (w / WPB) + r16, gc0 = 4 * (w % WPB) + g4;
    uint4 graw[CPL][GV];
    float gh = 0.f;
    if (narrow) {
        tq.load(q + base, rstride, valid, dio);
        tk.load(k + base, rstride, valid, dio);
    } else {
        tq.load(q + base, rstride, valid);
        tk.load(k + base, rstride, valid);
    }
    if constexpr (GH) {
        gh = reinterpret_cast<const float*>(g)[bbase + (size_t)min(grow, valid - 1) * H];
    } else {
        const TG* gp = g + base + (size_t)min(grow, valid - 1) * rstride;
#pragma unroll
        for (int cp = 0; cp < CPL; ++cp) {
            const int c8 = 8 * (gc0 + 4 * WPB * cp), cc = NARROW_OK ? min(c8, dio - 8) : c8;
#pragma unroll
            for (int vq = 0; vq < GV; ++vq) graw[cp][vq] = *reinterpret_cast<const uint4*>(gp + cc + GE * vq);
        }
    }
    const float braw = ld1<ST>(beta + bbase + (size_t)min(tid, valid - 1) * H);
    if constexpr (WITH_V) {
        __builtin_amdgcn_s_barrier();
        if (narrow)
            tv.load(v + base, rstride, valid, dio);
        else
            tv.load(v + base, rstride, valid);
    }
    tq.store(&s.ql[0][0], ChunkSmem<D, ST>::LDK);
    tk.store(&s.kr[0][0], ChunkSmem<D, ST>::LDK);
    int flag = 0;
#pragma unroll
    for (int cp = 0; cp < CPL; ++cp) {
        float x[8];
        const bool cok = !NARROW_OK || 8 * (gc0 + 4 * WPB * cp) < dio;
        if constexpr (GH) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = (grow < valid) ? gh : 0.f;
        } else {
#pragma unroll
            for (int vq = 0; vq < GV; ++vq) {
                const Vec16<TGE> xv{graw[cp][vq]};
#pragma unroll
                for (int e = 0; e < GE; ++e) x[GE * vq + e] = (grow < valid && cok) ? xv.get(e) : 0.f;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (!(x[e] <= 0.f)) flag = 1;
            x[e] = row16_scan(x[e]);
        }
        float* dst = &s.g[grow][8 * (gc0 + 4 * WPB * cp)];
        *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(x[4], x[5], x[6], x[7]);
    }
    if (tid < C) s.beta[tid] = (tid < valid) ? braw : 0.f;
    __syncthreads();
    return flag;
}

// OR of x over the workgroup through one LDS word (*w, zeroed by the caller
// before an earlier barrier).  Ends with a barrier.  The result is returned
// through readfirstlane, so the compiler knows it is uniform and branches on
// it with scalar branches.
// The wave's OR is formed bit by bit with ballots (one compare each, no LDS
// round trip); x must fit in NBITS bits.
template <int NTH, int NBITS = 9>
__device__ __forceinline__ int block_or(int x, int* w) {
    int wm = 0;
#pragma unroll
    for (int b = 0; b < NBITS; ++b)
        if (__ballot((x >> b) & 1)) wm |= 1 << b;
    if ((threadIdx.x & 63) == 0 && wm) atomicOr(w, wm);
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*w);
}

// Factor tables and the decay flags, from a (the in-block cumsums) and the
// load's g > 0 / NaN flag.  Returns, uniform over the workgroup, bit 4 set when
// the chunk must be evaluated pair by pair (g > 0 or NaN), bit i (0..3) set
// when diagonal block i's span exceeds SPAN_MAX, and bit 5 + i set when one of
// that block's 4-row sub-blocks does too (see subanchor_tile).  flagw: one
// zeroed LDS word.
template <int D, typename ST, int PREC, int NTH = 256>
__device__ __forceinline__ int chunk_factors2(ChunkSmem<D, ST>& s, int flag, int* flagw) {
    constexpr int TPC = NTH / D;   // threads per channel
    static_assert(TPC >= 1 && NTH % D == 0, "whole channels per workgroup");
    const int tid = threadIdx.x, d = tid % D;
    // whole waves per table row where D is a multiple of the wave size: the row
    // selects below are then scalar
    const int r = (D % 64 == 0) ? __builtin_amdgcn_readfirstlane(tid / D) : tid / D;
    int m = flag ? 16 : 0;
    // the channel's four block totals and (one thread per block, TPC >= NB) the
    // block's sub-block ends, all read together
    const float T0 = s.g[BS - 1][d], T1 = s.g[2 * BS - 1][d], T2 = s.g[3 * BS - 1][d], T3 = s.g[4 * BS - 1][d];
    const int ib = (r < NB) ? r : NB - 1;
    const float e0 = s.g[BS * ib + 3][d], e1 = s.g[BS * ib + 7][d], e2 = s.g[BS * ib + 11][d];
    const float T12 = T1 + T2;
    // table rows r, r + TPC, ...: exponents are sums of block totals (FAC_*)
    for (int row = r; row < FAC_ONE; row += TPC) {
        const float x = (row == 0) ? T0 : (row == 1) ? T0 + T1 : (row == 2) ? (T0 + T1) + T2
                      : (row == 3) ? T1 + (T2 + T3) : (row == 4) ? T2 + T3 : (row == 5) ? T3
                      : (row == 6) ? T1 : (row == 7) ? T2 : (row == 8) ? T12
                      : fminf(-((row == 9) ? T0 : (row == 10) ? T1 : (row == 11) ? T2 : T3), SPAN_MAX);
        s.fac[row][d] = kexp<PREC>(x);
    }
    if (r == TPC - 1) s.fac[FAC_ONE][d] = 1.f;
    // span guards of blocks r, r + TPC, ...: the whole block and its 4-row sub-blocks
    for (int i = r; i < NB; i += TPC) {
        const float T = (i == 0) ? T0 : (i == 1) ? T1 : (i == 2) ? T2 : T3;
        if (!(-T <= SPAN_MAX)) m |= 1 << i;
        const bool pre = TPC >= NB;   // this thread's only block, read above
        const float c0 = pre ? e0 : s.g[BS * i + 3][d], c1 = pre ? e1 : s.g[BS * i + 7][d];
        const float c2 = pre ? e2 : s.g[BS * i + 11][d];
        if (!(-c0 <= SUB_SPAN_MAX) || !(c0 - c1 <= SUB_SPAN_MAX) || !(c1 - c2 <= SUB_SPAN_MAX) ||
            !(c2 - T <= SUB_SPAN_MAX))
            m |= 32 << i;
    }
    return block_or<NTH>(m, flagw);
}

// The diagonal tile (i, i) of K K^T . e^{a_t - a_s} (and, with WITH_Q, of
// Q K^T . e^{a_t - a_s}) for a block whose 16-row span exceeds SPAN_MAX, from
// the raw rows of k (kr) and q (ql) and a, by one wave, before the transform.
// Anchors r_p = 16 i + 4 p - 1 (a_{16i-1} = 0) split the block into 4-row
// sub-blocks; pass p multiplies rows t of sub-block p, K_t e^{a_t - a_{r_p}}
// (<= 1), with rows s of sub-blocks <= p, K_s e^{a_{r_p} - a_s} (<= 1 before
// sub-block p, <= e^{4-row span} inside it), and the four passes accumulate
// into one tile (a pass contributes only to its own rows).  Valid when every
// 4-row span is <= SPAN_MAX.  Lane (g, n) holds rows 4 g .. 4 g + 3, column n
// of the tile; entries above the diagonal are not masked.  With ksel >= 0 only
// the 32 channels of k-step ksel contribute (a partial product, so that two
// waves can share a tile).
template <int D, typename ST, int PREC, bool WITH_Q>
__device__ __forceinline__ void subanchor_tile(const ChunkSmem<D, ST>& s, int i, f32x4& P, f32x4& Q, int ksel = -1) {
    const int l = lane_id(), r16 = l & 15, g4 = l >> 4, q = r16 >> 2;
    const int row = BS * i + r16;
    P = zero4();
    Q = zero4();
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        if (ksel >= 0 && ks != ksel) continue;
        float kv[8], qv[8], av[8], ar[NB][8], arq[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = 32 * ks + 16 * h + 4 * g4;
            const float4 k4 = ld4<ST>(&s.kr[row][c]), q4 = ld4<ST>(&s.ql[row][c]);
            const float4 a4 = *reinterpret_cast<const float4*>(&s.g[row][c]);
            kv[4 * h] = k4.x; kv[4 * h + 1] = k4.y; kv[4 * h + 2] = k4.z; kv[4 * h + 3] = k4.w;
            qv[4 * h] = q4.x; qv[4 * h + 1] = q4.y; qv[4 * h + 2] = q4.z; qv[4 * h + 3] = q4.w;
            av[4 * h] = a4.x; av[4 * h + 1] = a4.y; av[4 * h + 2] = a4.z; av[4 * h + 3] = a4.w;
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const float4 r4 = p ? *reinterpret_cast<const float4*>(&s.g[BS * i + 4 * p - 1][c])
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
                ar[p][4 * h] = r4.x; ar[p][4 * h + 1] = r4.y; ar[p][4 * h + 2] = r4.z; ar[p][4 * h + 3] = r4.w;
            }
            // the anchor of the lane's own sub-block, read by row (a pick among the
            // four loaded above compiles to branches per element); q = 0 reads a row
            // of the block and takes 0
            const float4 o4 = *reinterpret_cast<const float4*>(&s.g[BS * i + 4 * q - (q ? 1 : 0)][c]);
            arq[4 * h] = q ? o4.x : 0.f; arq[4 * h + 1] = q ? o4.y : 0.f;
            arq[4 * h + 2] = q ? o4.z : 0.f; arq[4 * h + 3] = q ? o4.w : 0.f;
        }
        float ea[8];   // e^{a_t - a_{r_q}}, the lane's row in its own sub-block q
#pragma unroll
        for (int e = 0; e < 8; ++e) ea[e] = kexp<PREC>(av[e] - arq[e]);
        // the lane's A operands, packed once; pass p keeps them on sub-block p's
        // rows only, and B on the rows of sub-blocks <= p (zeros picked after the
        // packing, a register at a time: past p the exponent is positive and may
        // overflow, and the pick drops that value)
        float ka[8], qa[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            ka[e] = kv[e] * ea[e];
            qa[e] = qv[e] * ea[e];
        }
        const Frag8 FA = frag_from_f32<PREC>(ka);
        Frag8 FQ{};
        if constexpr (WITH_Q) FQ = frag_from_f32<PREC>(qa);
        const Frag8 Z{};
#pragma unroll
        for (int p = 0; p < NB; ++p) {
            float bb[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) bb[e] = kv[e] * kexp<PREC>(ar[p][e] - av[e]);
            const Frag8 B = (q <= p) ? frag_from_f32<PREC>(bb) : Z;
            P = mma<PREC>((q == p) ? FA : Z, B, P);
            if constexpr (WITH_Q) Q = mma<PREC>((q == p) ? FQ : Z, B, Q);
        }
    }
}

// gamma_t of row t, channel d, from a (any chunk): a_t plus the totals of the
// blocks before t's
template <int D, typename ST>
__device__ __forceinline__ float chunk_gamma(const ChunkSmem<D, ST>& s, int t, int d) {
    float x = s.g[t][d];
    if (t >= BS) x += s.g[BS - 1][d];
    if (t >= 2 * BS) x += s.g[2 * BS - 1][d];
    if (t >= 3 * BS) x += s.g[3 * BS - 1][d];
    return x;
}

// Register-resident inverses of the four 16x16 diagonal blocks of I + L,
// L[t][s] = beta_t Akk[t][s]: wave w inverts block w by forward substitution,
// x_t = [t == c] - beta_t sum_{s<t} Akk[t][s] x_s for column c.  Lane
// (c = l / 4, p = l % 4) owns column c and the quarter s = 4 p .. 4 p + 3 of
// each row sum; the four partial sums of a column meet by two quad-permute
// DPP adds, so every step is a handful of dependent VALU operations on all 64
// lanes.  The block's rows are read before the substitution starts (one
// 16-byte read per row and lane, the same for the 16 lanes of a quarter);
// akk must hold zeros on and above the block's diagonal, as every writer of
// A_kk stores them.
// With fc != nullptr the block's transpose is also written as split (PREC 3)
// MFMA A fragments, fc[64 w + lane] = fragment of lane (g, r) holding
// T_ww[4g + e][r], so that other waves load it with one 16-byte read per lane.
template <int LDA>
__device__ __forceinline__ void diag_inverse_reg(const float* __restrict__ akk, const float* __restrict__ beta,
                                                 float (*tii)[BS][BS + 4], Frag4* fc = nullptr) {
    static_assert(BS == 16, "four quarters of four");
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l >> 2, p = l & 3;
    const float* Ab = akk + (size_t)(BS * w) * LDA + BS * w + 4 * p;
    float4 R[BS];   // R[t] = Akk[t][4 p .. 4 p + 3] of the block (zero at s >= t in akk)
    float bt[BS];
#pragma unroll
    for (int t = 1; t < BS; ++t) {
        bt[t] = beta[BS * w + t];
        R[t] = *reinterpret_cast<const float4*>(Ab + t * LDA);
    }
    __builtin_amdgcn_sched_barrier(0);
    float xq[4] = {0.f, 0.f, 0.f, 0.f};   // x_{4p} .. x_{4p+3}
    if (p == 0) xq[0] = (c == 0) ? 1.f : 0.f;
#pragma unroll
    for (int t = 1; t < BS; ++t) {
        float part = R[t].x * xq[0] + R[t].y * xq[1];
        part += R[t].z * xq[2] + R[t].w * xq[3];
        part += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0xB1, 0xf, 0xf, false));
        part += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0x4E, 0xf, 0xf, false));
        const float xt = ((t == c) ? 1.f : 0.f) - bt[t] * part;
        if ((t >> 2) == p) xq[t & 3] = xt;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tii[w][4 * p + e][c] = xq[e];
    if (fc) fc[64 * w + 16 * p + c] = frag4_from_f32<3>(xq);
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
