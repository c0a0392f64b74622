// kda_bwdw.hip -- the local-adjoint kernel of the KDA backward at D = 128.
//
// kda_bwd_localw_kernel: one 512-thread workgroup per chunk; wave w owns
// channel tile w (16 channels) of every per-(t, d) adjoint.  Same chunk
// algebra as the D = 64 kernels (nope_gdn_mlx.py:2579-2720, the transposed WY
// solve 1209-1286, the M backward kernels 2080-2295, the in-chunk reverse
// cumsum 2573-2577), with an LDS plan that fits D = 128:
//   - the chunk's operands that are read as fragments (dO, V', dV', h, dh, W,
//     U) come straight from global memory (L2): nothing of them is staged;
//   - A_kk and the inverted diagonal blocks of I + L come from the prep's
//     workspace, V' from the state recompute's;
//   - the anchored decay operands of phase 4 (k e^{gamma_t - gamma_r},
//     q e^{...}, k e^{gamma_r - gamma_t}, r the first row of t's 16-row block)
//     are the lane's own rows of its own channel, so they live in registers;
//   - dR = (I + L)^-T [dW | dU] passes through LDS one half (dW columns, then
//     dU columns) at a time.
// LDS: gamma and its factor tables, dP / dA (C x C fp32 each), half of dR, the
// diagonal inverses, the dbeta partials: about 118 KB.
#include "kda_internal.h"

namespace kda {

namespace {

template <int D>
struct WideLds {
    float g[C][D + 4];   // gamma, the in-chunk cumsum of g
    float er[NB][D];     // e^{gamma_16i}
    float f[6][D];       // e^{gamma_16i - gamma_16j}, pair_idx(i, j)
    float tot[NB][D];    // block totals of the cumsum
    float beta[C];
};

// rows of a (B, T, H, D) tensor as an fp32-valued A operand; rows at or past
// `valid` and the k-steps at or past `kvalid` (a multiple of 32) read as zero
template <typename TI>
__device__ __forceinline__ Fr8 rows8(const TI* base, size_t rstride, int row0, int k0, int valid, int kvalid) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    Fr8 f;
    if (row0 + r < valid && k0 < kvalid) {
        const TI* p = base + (size_t)(row0 + r) * rstride + k0 + 4 * g;
        const float4 x = ld4<TI>(p), y = ld4<TI>(p + 16);
        f.v[0] = x.x; f.v[1] = x.y; f.v[2] = x.z; f.v[3] = x.w;
        f.v[4] = y.x; f.v[5] = y.y; f.v[6] = y.z; f.v[7] = y.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f.v[e] = 0.f;
    }
    return f;
}

__device__ __forceinline__ float sum16w(float x) {
    x += __shfl_xor(x, 1, 64);
    x += __shfl_xor(x, 2, 64);
    x += __shfl_xor(x, 4, 64);
    x += __shfl_xor(x, 8, 64);
    return x;
}
__device__ __forceinline__ float sum4gw(float x) {
    x += __shfl_xor(x, 16, 64);
    x += __shfl_xor(x, 32, 64);
    return x;
}

// The diagonal tile of block m, pair by pair, for the lane's rows t = 16 m +
// 4 g4 + e of channel d: everything from LDS -- gamma g (row stride ldg), the
// staged raw k / q rows sk / sq (row stride ldq), dP sp and dA sda (row stride
// lda) -- and the sums (dk, dq, dgamma terms) to res[3][16][D].  Not inlined:
// its loops stay out of the register allocation of the kernel's common path.
template <int D, typename TI, int PREC>
__device__ __noinline__ void wide_pair_block(const float* __restrict__ g, int ldg, const TI* __restrict__ sk,
                                             const TI* __restrict__ sq, int ldq, const float* __restrict__ sp,
                                             const float* __restrict__ sda, int lda, float* __restrict__ res, int m,
                                             int g4, int d) {
    // the lane's four rows advance together: four independent sums per step
    float gt[4], kt[4], qt[4], ak[4], aq[4], ag[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = BS * m + 4 * g4 + e;
        gt[e] = g[t * ldg + d];
        kt[e] = ld1<TI>(sk + t * ldq + d);
        qt[e] = ld1<TI>(sq + t * ldq + d);
        ak[e] = aq[e] = ag[e] = 0.f;
    }
#pragma unroll 1
    for (int r = 0; r < BS; ++r) {
        const int sx = BS * m + r;
        const float gs = g[sx * ldg + d], ks_raw = ld1<TI>(sk + sx * ldq + d), qs_raw = ld1<TI>(sq + sx * ldq + d);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int rt = 4 * g4 + e, t = BS * m + rt;
            // row side: pair (t, s), s < t; column side: pair (s, t), s > t
            const bool row = r < rt, col = r > rt;
            const float ex = kexp<PREC>(row ? gt[e] - gs : gs - gt[e]);
            const float pp = sp[row ? t * lda + sx : sx * lda + t], pa = sda[row ? t * lda + sx : sx * lda + t];
            const float ks = ks_raw * ex;
            const float c = (pp * ks_raw + pa * qs_raw) * ex;
            ak[e] += row ? pp * ks : col ? c : 0.f;
            aq[e] += row ? pa * ks : 0.f;
            ag[e] += row ? (pp * kt[e] + pa * qt[e]) * ks : col ? -c * kt[e] : 0.f;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int rt = 4 * g4 + e;
        res[(0 * BS + rt) * D + d] = ak[e];
        res[(1 * BS + rt) * D + d] = aq[e];
        res[(2 * BS + rt) * D + d] = ag[e];
    }
}

}  // namespace

template <int D, typename TI, typename TG, int PREC>
__global__ __launch_bounds__(4 * D) void kda_bwd_localw_kernel(const LocalArgs a) {
    constexpr int NT = D / BS, NTH = 4 * D, NW = NTH / 64;
    static_assert(NW == NT && NB == 4, "one wave per channel tile, one thread per (channel, row block)");
    __shared__ WideLds<D> s;
    __shared__ __align__(16) float sp[C][C + 4];   // Akk, then dP = diag(beta) dL
    __shared__ float sda[C][C + 4];         // dAqk (lower, with the diagonal)
    __shared__ __align__(16) float tii[NB][BS][BS + 4];
    __shared__ float sdb[NB + NT][C];       // dbeta partials: [j] from dL tiles of column block j, [NB + nt] channel tile nt
    __shared__ __align__(16) char pfbuf[256];   // landing bytes of the L2 prefetch
    // Staging area.  bf16 (STG): the chunk's raw k and q rows (phase 0 to the
    // per-lane values), then dO, V', dV' and v (phase 1 and the dA tiles), then one
    // half of dR (fp32) beside W or U (phases 2-3), each brought in with
    // coalesced 16-byte loads so that fragments and per-lane values are LDS
    // reads.  fp32 (no room for the staged tiles): dR only; the rest is read
    // from global memory.
    constexpr bool STG = sizeof(TI) == 2;
    constexpr int LDQ = D + 8, LDR = D + 4;   // bf16 rows with a 16-byte pad; fp32 dR rows
    constexpr int T_BYTES = C * LDQ * (int)sizeof(TI), R_BYTES = C * LDR * 4;
    constexpr int STG_BYTES = STG ? ((4 * T_BYTES > R_BYTES + T_BYTES) ? 4 * T_BYTES : R_BYTES + T_BYTES) : R_BYTES;
    __shared__ __align__(16) unsigned char stg[STG_BYTES];
    float* sdr = reinterpret_cast<float*>(stg);                      // [C][LDR], one half of dR: dR_k, then dR_v
    TI* const st0 = reinterpret_cast<TI*>(stg);                       // k | dO
    TI* const st1p = reinterpret_cast<TI*>(stg + T_BYTES);            // q | V'
    TI* const st2 = reinterpret_cast<TI*>(stg + 2 * T_BYTES);         // dV'
    TI* const st3 = reinterpret_cast<TI*>(stg + 3 * T_BYTES);         // v
    TI* const swu = reinterpret_cast<TI*>(stg + R_BYTES);             // W, then U (beside dR)

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15,
              g4 = l >> 4;
    __builtin_assume(w >= 0 && w < NW);
    const int ch = blockIdx.x, bh = ch / a.nc, n = ch - bh * a.nc;
    const int b = bh / a.H, h = bh - b * a.H;
    const int t0 = n * C, valid = min(C, a.T - t0);
    // dio: the channels of a q, k, v, g, dout, dq, dk, dv, dg row (< D for a
    // narrower head: the rest read as zero and are not written)
    const int dio = a.dio > 0 ? a.dio : D;
    const bool narrow = dio < D;
    const size_t rs = (size_t)a.H * dio;
    const size_t base = ((size_t)b * a.T + t0) * rs + (size_t)h * dio;
    const size_t bbase = ((size_t)b * a.T + t0) * a.H + h;
    const TI* q = static_cast<const TI*>(a.q);
    const TI* k = static_cast<const TI*>(a.k);
    const TI* v = static_cast<const TI*>(a.v);
    const TG* g = static_cast<const TG*>(a.g);
    const TI* beta = static_cast<const TI*>(a.beta);
    const TI* dout = static_cast<const TI*>(a.dout);
    const size_t cCD = (size_t)ch * C * D, cCC = (size_t)ch * C * C;
    const TI* hS = static_cast<const TI*>(a.h) + (size_t)ch * D * D;
    const TI* dhS = static_cast<const TI*>(a.dh) + (size_t)ch * D * D;
    const TI* Vp = static_cast<const TI*>(a.Vp) + cCD;
    const TI* dVp = static_cast<const TI*>(a.dVp) + cCD;
    const TI* Wc = static_cast<const TI*>(a.W) + cCD;
    const TI* Uc = static_cast<const TI*>(a.U) + cCD;

    // ---------------- phase 0: A_kk, inverses, gamma, factors ----------------
    // every load of the phase issued before any is used: A_kk and the inverses
    // as 16-byte pieces, g of the thread's 16 rows, k and q rows (bf16)
    constexpr int AKV = C * C / 4, TIV = NB * BS * BS / 4;
    float4 akv[(AKV + NTH - 1) / NTH];
#pragma unroll
    for (int i = 0; i < (AKV + NTH - 1) / NTH; ++i)
        if (AKV % NTH == 0 || tid + NTH * i < AKV)
            akv[i] = reinterpret_cast<const float4*>(a.Akk + cCC)[tid + NTH * i];
    float4 tiv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < TIV) tiv = reinterpret_cast<const float4*>(a.Tii + (size_t)ch * NB * BS * BS)[tid];
    const int cd = tid % D, cb = tid / D;
    // rows past T (and channels past dio) are read from the last valid row
    // (channel) -- no branch around a load, so the sixteen loads are in flight
    // together -- and zeroed below
    float gx[BS];
    const int cdl = min(cd, dio - 1);
#pragma unroll
    for (int r = 0; r < BS; ++r) {
        const int t = BS * cb + r;
        gx[r] = ld1<TG>(g + base + (size_t)min(t, valid - 1) * rs + cdl);
    }
    Tile<TI, C, D, NTH> tkr, tqr;
    if constexpr (STG) {
        if (narrow) {
            tkr.load(k + base, rs, valid, dio);
            tqr.load(q + base, rs, valid, dio);
        } else {
            tkr.load(k + base, rs, valid);
            tqr.load(q + base, rs, valid);
        }
    }
#pragma unroll
    for (int i = 0; i < (AKV + NTH - 1) / NTH; ++i)
        if (AKV % NTH == 0 || tid + NTH * i < AKV) {
            const int e = 4 * (tid + NTH * i);
            *reinterpret_cast<float4*>(&sp[e / C][e % C]) = akv[i];
        }
    if (tid < TIV) {
        const int e = 4 * tid, i = e / (BS * BS), r = (e / BS) % BS, c = e % BS;
        *reinterpret_cast<float4*>(&tii[i][r][c]) = tiv;
    }
    for (int idx = tid; idx < (NB + NT) * C; idx += NTH) sdb[idx / C][idx % C] = 0.f;
    if (tid < C) s.beta[tid] = (tid < valid) ? ld1<TI>(beta + bbase + (size_t)tid * a.H) : 0.f;
    if constexpr (STG) {
        tkr.store(st0, LDQ);
        tqr.store(st1p, LDQ);
    }
    // thread (channel cd, block cb): inclusive cumsum of g over the block's 16
    // rows (rows past T are g = 0: no decay), then the totals of earlier blocks
    // flag: g > 0 or a NaN somewhere (every pair of the chunk pair by pair);
    // sflag: a 16-row block's decay span beyond the anchored guard (its
    // diagonal tile pair by pair, the other tiles on exact per-lane factors)
    int flag = 0, sflag = 0;
    {
        float run = 0.f;
#pragma unroll
        for (int r = 0; r < BS; ++r) {
            const int t = BS * cb + r;
            const float x = (t < valid && cd < dio) ? gx[r] : 0.f;
            if (!(x <= 0.f)) flag = 1;
            run += x;
            s.g[t][cd] = run;
        }
        s.tot[cb][cd] = run;
        __syncthreads();
        float off = 0.f;
        for (int bb = 0; bb < cb; ++bb) off += s.tot[bb][cd];
        if (cb > 0)
#pragma unroll 4
            for (int r = 0; r < BS; ++r) s.g[BS * cb + r][cd] += off;
    }
    __syncthreads();
    // factor tables and the span guard (a chunk beyond it, or with g > 0 or a
    // NaN, is evaluated pair by pair)
    for (int idx = tid; idx < NB * D; idx += NTH) {
        const int j = idx / D, d = idx % D;
        if (!(s.g[BS * j][d] - s.g[BS * j + BS - 1][d] <= SPAN_MAX)) sflag = 1;
        s.er[j][d] = kexp<PREC>(s.g[BS * j][d]);
    }
    for (int idx = tid; idx < 6 * D; idx += NTH) {
        const int p = idx / D, d = idx % D;
        const int i = (p >= 3) ? 3 : (p >= 1) ? 2 : 1, j = p - pair_idx(i, 0);
        s.f[p][d] = kexp<PREC>(s.g[BS * i][d] - s.g[BS * j][d]);
    }
    const int unsafe = __syncthreads_or(flag);
    const int strong = __syncthreads_or(sflag);

    // wave w owns channel tile w: rows t = 16 m + 4 g4 + e, channel d
    const int nt = w, d = nt * BS + r16;
    // raw k, q of the lane's rows; el = e^{gamma_t - gamma_r} (r = 16 m), eb =
    // e^{G - gamma_t}, erb = e^{gamma_r}
    float kx[NB][4], qx[NB][4], el[NB][4], eb[NB][4], erb[NB];
    {
        const float G = s.g[C - 1][d];
#pragma unroll
        for (int m = 0; m < NB; ++m) {
            const float gr = s.g[BS * m][d];
            erb[m] = s.er[m][d];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                const float gt = s.g[t][d];
                if constexpr (STG) {
                    kx[m][e] = ld1<TI>(st0 + t * LDQ + d);
                    qx[m][e] = ld1<TI>(st1p + t * LDQ + d);
                } else {
                    // clamped row and channel, selected after the load: no branch around it
                    const size_t oc = base + (size_t)min(t, valid - 1) * rs + min(d, dio - 1);
                    const float kv = ld1<TI>(k + oc), qv = ld1<TI>(q + oc);
                    kx[m][e] = (t < valid && d < dio) ? kv : 0.f;
                    qx[m][e] = (t < valid && d < dio) ? qv : 0.f;
                }
                el[m][e] = kexp<PREC>(gt - gr);
                eb[m][e] = kexp<PREC>(G - gt);
            }
        }
    }

    f32x4 dqa[NB], dka[NB], dga[NB], dWt[NB];
#pragma unroll
    for (int m = 0; m < NB; ++m) { dqa[m] = zero4(); dka[m] = zero4(); dga[m] = zero4(); dWt[m] = zero4(); }
    float dgcol = 0.f;

    // ---------------- phase 1: products over dv ----------------
    // bf16: dO, V', dV' staged (the k, q rows are in registers now); the B
    // operands, rows of h and dh of the wave's own channel tile, straight from
    // global memory, once
    Frag8 Bh[STG ? D / 32 : 1], Bdh[STG ? D / 32 : 1];
    if constexpr (STG) {
        Tile<TI, C, D, NTH> tdo, tvp, tdvp, tvv;
        if (narrow)
            tdo.load(dout + base, rs, valid, dio);
        else
            tdo.load(dout + base, rs, valid);
        tvp.load(Vp, D);
        tdvp.load(dVp, D);
        if (narrow)
            tvv.load(v + base, rs, valid, dio);
        else
            tvv.load(v + base, rs, valid);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            Bh[ks] = ldfrag_c<1, TI>(hS, D, BS * nt, 32 * ks);
            Bdh[ks] = ldfrag_c<1, TI>(dhS, D, BS * nt, 32 * ks);
        }
        __syncthreads();   // every lane's k, q reads are done
        tdo.store(st0, LDQ);
        tvp.store(st1p, LDQ);
        tdvp.store(st2, LDQ);
        tvv.store(st3, LDQ);
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < NB; ++m) {
        f32x4 dQp = zero4(), dKb = zero4(), dW = zero4();
        if constexpr (STG) {
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                dQp = mma<1>(ldfrag_c<1, TI>(st0, LDQ, BS * m, 32 * ks), Bh[ks], dQp);
                dKb = mma<1>(ldfrag_c<1, TI>(st1p, LDQ, BS * m, 32 * ks), Bdh[ks], dKb);
                dW = mma<1>(ldfrag_c<1, TI>(st2, LDQ, BS * m, 32 * ks), Bh[ks], dW);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) dW[e] = -dW[e];
        } else {
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                const Fr8 Bh8 = frag8(hS, D, BS * nt, 32 * ks);
                const Fr8 Bdh8 = frag8(dhS, D, BS * nt, 32 * ks);
                dQp = mma8<PREC>(rows8<TI>(dout + base, rs, BS * m, 32 * ks, valid, dio), Bh8, dQp);
                dKb = mma8<PREC>(frag8(Vp, D, BS * m, 32 * ks), Bdh8, dKb);
                dW = mma8<PREC>(neg(frag8(dVp, D, BS * m, 32 * ks)), Bh8, dW);
            }
        }
        dWt[m] = dW;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float egt = erb[m] * el[m][e];                 // e^{gamma_t}
            dqa[m][e] = dQp[e] * egt;
            dka[m][e] = dKb[e] * eb[m][e];
            const float kbv = kx[m][e] * eb[m][e];
            dga[m][e] = dQp[e] * qx[m][e] * egt - dKb[e] * kbv;
            dgcol += dKb[e] * kbv;
        }
    }
    {
        // state-decay term of dG: e^G sum_col dh[d][col] h[d][col]
        float part = 0.f;
        float4 xh[D / 16], xd[D / 16];
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
            xh[c] = ld4<TI>(hS + (size_t)d * D + g4 * (D / 4) + 4 * c);
            xd[c] = ld4<TI>(dhS + (size_t)d * D + g4 * (D / 4) + 4 * c);
        }
#pragma unroll
        for (int c = 0; c < D / 16; ++c)
            part += (xd[c].x * xh[c].x + xd[c].y * xh[c].y) + (xd[c].z * xh[c].z + xd[c].w * xh[c].w);
        dgcol = sum4gw(dgcol) + kexp<PREC>(s.g[C - 1][d]) * sum4gw(part);
    }
    // dAqk = tril(dO V'^T), 10 lower tiles over the waves
    for (int tix = w; tix < 10; tix += NW) {
        int i, j;
        tile_ij(tix, i, j);
        f32x4 acc = zero4();
        if constexpr (STG) {
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                acc = mma<1>(ldfrag_c<1, TI>(st0, LDQ, BS * i, 32 * ks), ldfrag_c<1, TI>(st1p, LDQ, BS * j, 32 * ks), acc);
        } else {
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                acc = mma8<PREC>(rows8<TI>(dout + base, rs, BS * i, 32 * ks, valid, dio),
                                 frag8(Vp, D, BS * j, 32 * ks), acc);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
            sda[t][sx] = (sx <= t) ? acc[e] : 0.f;
        }
    }
    // the lane's dV' and v values for the solve (bf16: from the staged tiles,
    // before the barrier below frees them)
    f32x4 dvp[NB], vx[NB];
#pragma unroll
    for (int m = 0; m < NB; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * m + 4 * g4 + e;
            if constexpr (STG) {
                dvp[m][e] = ld1<TI>(st2 + t * LDQ + d);
                vx[m][e] = ld1<TI>(st3 + t * LDQ + d);
            } else {
                dvp[m][e] = ld1<TI>(dVp + (size_t)t * D + d);
                const float vv = ld1<TI>(v + base + (size_t)min(t, valid - 1) * rs + min(d, dio - 1));
                vx[m][e] = (t < valid && d < dio) ? vv : 0.f;
            }
        }
    // zero upper tiles of sda
    for (int idx = tid; idx < 6 * BS * BS; idx += NTH) {
        const int tile = idx / (BS * BS), e = idx - tile * BS * BS;
        const int i = (tile < 3) ? 0 : (tile < 5) ? 1 : 2;
        const int j = (tile < 3) ? tile + 1 : (tile < 5) ? tile - 1 : 3;
        sda[BS * i + e / BS][BS * j + (e % BS)] = 0.f;
    }
    __syncthreads();

    // ---------------- phase 2: transposed WY solve (fp32-accurate split products) ----------------
    f32x4 dRk[NB], dRv[NB];
    Tile<TI, C, D, NTH> tw, tu;
    {
#pragma unroll
        for (int i = NB - 1; i >= 0; --i) {
            f32x4 Yk = dWt[i], Yv = dvp[i];
#pragma unroll
            for (int j = i + 1; j < NB; ++j) {
                // A[a][b] = -L[16j + b][16i + a] = -beta_{16j+b} Akk[16j+b][16i+a]
                Fr4 A;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int rb = BS * j + 4 * g4 + e;
                    A.v[e] = -s.beta[rb] * sp[rb][BS * i + r16];
                }
                Yk = mma4<3>(A, acc2frag4(dRk[j]), Yk);
                Yv = mma4<3>(A, acc2frag4(dRv[j]), Yv);
            }
            const Fr4 Tt = frag4T(&tii[i][0][0], BS + 4, 0, 0);     // A[a][b] = T_ii[b][a]
            dRk[i] = mma4<3>(Tt, acc2frag4(Yk), zero4());
            dRv[i] = mma4<3>(Tt, acc2frag4(Yv), zero4());
        }
        // bf16: W and U come to the staging area beside dR for phase 3 (loaded
        // here, after the solve's chain, and stored at its end)
        if constexpr (STG) {
            tw.load(Wc, D);
            tu.load(Uc, D);
        }
        TI* dv = static_cast<TI*>(a.dv);
#pragma unroll
        for (int m = 0; m < NB; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                const float bt = s.beta[t];
                const float egt = erb[m] * el[m][e];
                const float vv = vx[m][e];
                if (t < valid && d < dio) st1<TI>(dv + base + (size_t)t * rs + d, bt * dRv[m][e]);
                dka[m][e] += bt * egt * dRk[m][e];
                dga[m][e] += dRk[m][e] * bt * egt * kx[m][e];
                const float db = sum16w(dRv[m][e] * vv + dRk[m][e] * egt * kx[m][e]);
                if (r16 == 0) sdb[NB + nt][t] = db;
                sdr[t * LDR + d] = dRk[m][e];
            }
        }
    }
    if constexpr (STG) tw.store(swu, LDQ);
    __syncthreads();

    // L2 prefetch of the chunk this XCD starts next (chunk ids a CU count apart
    // go to one XCD and start about when this one ends): its phase-0 inputs --
    // the rows of q, k and g (two 128-byte lines a row) and A_kk and the
    // inverses -- one 4-byte DMA per line, the landing bytes scratch.  Issued
    // after this chunk's last global load, so that no wait of this chunk covers
    // it, and waited for at the end.  Waves 0-1 take q, 2-3 k, 4-5 g, 6-7 A_kk,
    // and 32 lanes of wave 0 the inverses (the pointer is picked per wave).
    if (a.pf_ahead > 0 && ch + a.pf_ahead < (int)gridDim.x) {
        const int pc = ch + a.pf_ahead, pbh = pc / a.nc, pn = pc - pbh * a.nc;
        const int pb = pbh / a.H, ph = pbh - pb * a.H, pvalid = min(C, a.T - pn * C);
        const size_t pbase = ((size_t)pb * a.T + (size_t)pn * C) * rs + (size_t)ph * dio;
        const uint32_t m = lds_addr(pfbuf);
        const int grp = w >> 1, li = tid & 127, r = li >> 1;
        const char* p = nullptr;
        if (grp == 3) {
            p = reinterpret_cast<const char*>(a.Akk + (size_t)pc * C * C) + 128 * li;
        } else if (r < pvalid) {
            const char* tp = static_cast<const char*>(grp == 0 ? a.q : grp == 1 ? a.k : a.g);
            const size_t es = (grp == 2) ? sizeof(TG) : sizeof(TI);
            p = tp + (pbase + (size_t)r * rs) * es + 128 * (li & 1);
        }
        if (p) dma4(p, m);
        if (w == 0 && l < 32) dma4(reinterpret_cast<const char*>(a.Tii + (size_t)pc * NB * BS * BS) + 128 * l, m);
    }

    // ---------------- phase 3: dL = -tril(dR [W | U]^T, -1), one half of dR at a time ----------------
    // bf16: W and U are exact in bf16, so splitting only dR (PREC 2) keeps the
    // product fp32-accurate; fp32: both split (PREC 3)
    constexpr int TPW = (10 + NW - 1) / NW;
    f32x4 accL[TPW];
    auto dl_half = [&](const TI* gX) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tix = w + NW * u;
            if (tix < 10) {
                int i, j;
                tile_ij(tix, i, j);
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    if constexpr (STG)
                        accL[u] = mma<2>(ldfrag_c<2, float>(sdr, LDR, BS * i, 32 * ks),
                                         ldfrag_c<1, TI>(swu, LDQ, BS * j, 32 * ks), accL[u]);
                    else
                        accL[u] = mma8<3>(frag8(sdr, LDR, BS * i, 32 * ks), frag8(gX, D, BS * j, 32 * ks), accL[u]);
                }
            }
        }
    };
#pragma unroll
    for (int u = 0; u < TPW; ++u) accL[u] = zero4();
    dl_half(Wc);
    __syncthreads();   // dR_k and W read by every wave
#pragma unroll
    for (int m = 0; m < NB; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) sdr[(BS * m + 4 * g4 + e) * LDR + d] = dRv[m][e];
    if constexpr (STG) tu.store(swu, LDQ);
    __syncthreads();
    dl_half(Uc);
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
        const int tix = w + NW * u;
        if (tix < 10) {
            int i, j;
            tile_ij(tix, i, j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
                const float dL = (sx < t) ? -accL[u][e] : 0.f;
                const float db = sum16w(dL * sp[t][sx]);
                if (r16 == 0) sdb[j][t] = db;
                sp[t][sx] = s.beta[t] * dL;
            }
        }
    }
    __syncthreads();

    // ---------------- phase 4: decay-masked K K^T / Q K^T adjoints ----------------
    // Anchored adjoints (g <= 0 everywhere).  STRONG: some 16-row block spans
    // more than SPAN_MAX, so the block-start anchor's factor e^{gamma_16j -
    // gamma_s} could overflow: the off-diagonal tiles take the exact per-lane
    // factor e^{gamma_16i - gamma_s} (<= 1) instead of er * F_ij, and the
    // diagonal tiles are evaluated pair by pair within their block.
    auto anchored = [&](auto strong_c) __attribute__((always_inline)) {
        constexpr bool STRONG = decltype(strong_c)::value;
        // row and column sides of a pair must agree to fp32: exact split products
        constexpr int PX = PREC >= 3 ? 4 : PREC;
        // er = e^{gamma_r - gamma_t} (r = 16 m), formed here rather than with the
        // other per-lane values so that it is not live across phases 1-3
        float er[NB][4];
        if constexpr (!STRONG) {
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                const float gr = s.g[BS * m][d];
#pragma unroll
                for (int e = 0; e < 4; ++e) er[m][e] = kexp<PREC>(gr - s.g[BS * m + 4 * g4 + e][d]);
            }
        }
        // STRONG: the exact factor e^{gamma_16i - gamma_s}, s = 16 j + 4 g4 + e,
        // j < i, formed where it is used (the same expression on both sides of
        // a pair, so both use the same value)
        auto wf = [&](int i, int j, int e) __attribute__((always_inline)) {
            return kexp<PREC>(s.g[BS * i][d] - s.g[BS * j + 4 * g4 + e][d]);
        };
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            f32x4 dKl = zero4(), dQl = zero4();
#pragma unroll
            for (int j = 0; j <= i; ++j) {
                if (STRONG && j == i) continue;
                const float fs = (j < i) ? s.f[pair_idx(i, j)][d] : 1.f;
                Fr4 B;   // K_r of the lane's rows of block j (channel d), times the pair's factor
#pragma unroll
                for (int e = 0; e < 4; ++e) B.v[e] = STRONG ? kx[j][e] * wf(i, j, e) : kx[j][e] * er[j][e] * fs;
                dKl = mma4<PX>(frag4(&sp[0][0], C + 4, BS * i, BS * j), B, dKl);
                Fr4 Aq = frag4(&sda[0][0], C + 4, BS * i, BS * j);
                if (j == i) {   // the diagonal pairs (t, t) are added apart, below
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * g4 + e == r16) Aq.v[e] = 0.f;
                }
                dQl = mma4<PX>(Aq, B, dQl);
            }
            Fr4 Bk, Bq;   // K_l, Q_l of the lane's rows of block i
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                Bk.v[e] = kx[i][e] * el[i][e];
                Bq.v[e] = qx[i][e] * el[i][e];
            }
            // each pair's row-t and column-s terms of dgamma cancel in the reverse
            // cumsum; weight each side by the operand values the other side's MFMA
            // used, so that the cancellation is exact to fp32
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dka[i][e] += dKl[e] * el[i][e];
                dqa[i][e] += dQl[e] * el[i][e];
                dga[i][e] += dKl[e] * mfma_operand<PREC>(Bk.v[e]) + dQl[e] * mfma_operand<PREC>(Bq.v[e]);
            }
#pragma unroll
            for (int j = 0; j <= i; ++j) {
                if (STRONG && j == i) continue;
                f32x4 dKr = mma4<PX>(frag4T(&sp[0][0], C + 4, BS * j, BS * i), Bk, zero4());
                Fr4 Aq = frag4T(&sda[0][0], C + 4, BS * j, BS * i);
                if (j == i) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * g4 + e == r16) Aq.v[e] = 0.f;
                }
                dKr = mma4<PX>(Aq, Bq, dKr);
                const float fs = (j < i) ? s.f[pair_idx(i, j)][d] : 1.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float ws = STRONG ? wf(i, j, e) : fs * er[j][e];
                    dka[j][e] += dKr[e] * ws;
                    // the row side's B operand for this s and block pair
                    dga[j][e] -= dKr[e] * mfma_operand<PREC>(STRONG ? kx[j][e] * ws : kx[j][e] * er[j][e] * fs);
                }
            }
        }
        if constexpr (STRONG) {
            // The diagonal tiles pair by pair within each block, with the exact
            // weight e^{gamma_t - gamma_s} (s < t) from LDS gamma.  Everything the
            // pair loops read comes from LDS -- the raw k and q rows (exact in
            // bf16) staged in the free staging area -- and their sums go back
            // there (per block: 16 rows x 3 planes, fp32), so the loops hold no
            // per-lane arrays; each lane then adds its own rows' sums.
            TI* const sk = st0;
            TI* const sq = st1p;
            float* const res = reinterpret_cast<float*>(stg + 2 * T_BYTES);   // [3][BS][D]
            static_assert(2 * T_BYTES + 3 * BS * D * 4 <= STG_BYTES, "pair sums fit the staging area");
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * m + 4 * g4 + e;
                    st1<TI>(sk + t * LDQ + d, kx[m][e]);
                    st1<TI>(sq + t * LDQ + d, qx[m][e]);
                }
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                __syncthreads();   // staged rows visible; the previous block's sums read
                wide_pair_block<D, TI, PREC>(&s.g[0][0], D + 4, sk, sq, LDQ, &sp[0][0], &sda[0][0], C + 4, res, m, g4,
                                             d);
                // the lane's own rows: written by itself above, no barrier needed
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int rt = 4 * g4 + e;
                    dka[m][e] += res[(0 * BS + rt) * D + d];
                    dqa[m][e] += res[(1 * BS + rt) * D + d];
                    dga[m][e] += res[(2 * BS + rt) * D + d];
                }
            }
        }
    };
    // (fp32 operands: no room to stage k and q, so a chunk past the span guard
    // takes the pair-by-pair path below)
    if (!unsafe && !(strong && !STG)) {
        if (STG && strong)
            anchored(std::integral_constant<bool, STG>{});
        else
            anchored(std::false_type{});
    } else {
        // pair by pair with the exact weight e^{gamma_t - gamma_s}: raw k and q of
        // the other rows from global memory, gamma from LDS
#pragma unroll
        for (int m = 0; m < NB; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                const float gt = s.g[t][d];
                float ak = 0.f, aq = 0.f, ag = 0.f;
                for (int sx = 0; sx < t; ++sx) {
                    const float ksx = (sx < valid && d < dio) ? ld1<TI>(k + base + (size_t)sx * rs + d) : 0.f;
                    const float ks = ksx * kexp<PREC>(gt - s.g[sx][d]);
                    const float pp = sp[t][sx], pa = sda[t][sx];
                    ak += pp * ks;
                    aq += pa * ks;
                    ag += (pp * kx[m][e] + pa * qx[m][e]) * ks;
                }
                for (int sx = t + 1; sx < C; ++sx) {
                    const float ksx = (sx < valid && d < dio) ? ld1<TI>(k + base + (size_t)sx * rs + d) : 0.f;
                    const float qsx = (sx < valid && d < dio) ? ld1<TI>(q + base + (size_t)sx * rs + d) : 0.f;
                    const float ex = kexp<PREC>(s.g[sx][d] - gt);
                    const float pp = sp[sx][t], pa = sda[sx][t];
                    const float c = (pp * ksx + pa * qsx) * ex;
                    ak += c;
                    ag -= c * kx[m][e];
                }
                dka[m][e] += ak;
                dqa[m][e] += aq;
                dga[m][e] += ag;
            }
        }
    }
    // the diagonal pairs (t, t) of A_qk (weight 1): dq_t += dA_tt k_t and
    // dk_t += dA_tt q_t, and nothing in dgamma_t (its row and column terms are
    // equal and opposite)
#pragma unroll
    for (int m = 0; m < NB; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * m + 4 * g4 + e;
            dqa[m][e] += sda[t][t] * kx[m][e];
            dka[m][e] += sda[t][t] * qx[m][e];
        }

    // ---------------- phase 5: dG, reverse cumsum, stores ----------------
    if (g4 == 3) dga[NB - 1][3] += dgcol;        // row C-1
    float lsum[NB][4], tots[NB];
#pragma unroll
    for (int m = 0; m < NB; ++m) {
        float run = 0.f;
#pragma unroll
        for (int e = 3; e >= 0; --e) { run += dga[m][e]; lsum[m][e] = run; }
        tots[m] = run;
    }
    float after_m = 0.f;   // sum over row tiles > m
#pragma unroll
    for (int m = NB - 1; m >= 0; --m) {
        const float t0v = __shfl(tots[m], r16, 64);
        const float t1v = __shfl(tots[m], r16 + 16, 64);
        const float t2v = __shfl(tots[m], r16 + 32, 64);
        const float t3v = __shfl(tots[m], r16 + 48, 64);
        const float later = (g4 < 1 ? t1v : 0.f) + (g4 < 2 ? t2v : 0.f) + (g4 < 3 ? t3v : 0.f);
#pragma unroll
        for (int e = 0; e < 4; ++e) lsum[m][e] += later + after_m;
        after_m += t0v + t1v + t2v + t3v;
    }
    TI* dq = static_cast<TI*>(a.dq);
    TI* dk = static_cast<TI*>(a.dk);
    TG* dg = static_cast<TG*>(a.dg);
#pragma unroll
    for (int m = 0; m < NB; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * m + 4 * g4 + e;
            if (t < valid && d < dio) {
                const size_t o = base + (size_t)t * rs + d;
                st1<TI>(dq + o, dqa[m][e]);
                st1<TI>(dk + o, dka[m][e]);
                st1<TG>(dg + o, lsum[m][e]);
            }
        }
    if (tid < valid) {
        float db = 0.f;
#pragma unroll
        for (int j = 0; j < NB + NT; ++j) db += sdb[j][tid];
        st1<TI>(static_cast<TI*>(a.dbeta) + bbase + (size_t)tid * a.H, db);
    }
    dma_wait<0>();   // the prefetch has landed before the workgroup's LDS is released
}

// bf16 operands: bf16 MFMA products (PREC 1); fp32: split-bf16 products
// accurate to fp32 (PREC 3)
hipError_t launch_local_wide(const LocalArgs& args, int D, int in_bf16, int g_bf16, int nchunks, hipStream_t st) {
    if (D != 128) return hipErrorInvalidValue;
    // prefetch distance: one chunk per CU (one workgroup fills a CU)
    int dev = 0;
    LocalArgs a = args;
    a.pf_ahead = (hipGetDevice(&dev) == hipSuccess) ? device_cu_count(dev) : 0;
    if (in_bf16) {
        if (g_bf16)
            hipLaunchKernelGGL((kda_bwd_localw_kernel<128, uint16_t, uint16_t, 1>), dim3(nchunks), dim3(512), 0, st, a);
        else
            hipLaunchKernelGGL((kda_bwd_localw_kernel<128, uint16_t, float, 1>), dim3(nchunks), dim3(512), 0, st, a);
    } else {
        if (g_bf16)
            hipLaunchKernelGGL((kda_bwd_localw_kernel<128, float, uint16_t, 3>), dim3(nchunks), dim3(512), 0, st, a);
        else
            hipLaunchKernelGGL((kda_bwd_localw_kernel<128, float, float, 3>), dim3(nchunks), dim3(512), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace kda
