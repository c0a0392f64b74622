// kda_bwd.hip -- backward kernels of the KDA chunkwise WY recurrence (gfx950).
//
// The backward stores no per-step state.  The forward's chunk-boundary states
// are recomputed (prep + kda_recur_kernel MODE 1), the reverse state carry
// (kda_dh_kernel, kda_recur.hip) stores dS at each chunk end and dV', then:
//
//   kda_bwd_local3_kernel (bf16 operands) / kda_bwd_local_kernel (fp32 operands)
//                     one workgroup per chunk, fully parallel: every remaining
//                     adjoint of the chunk -- output / state products, the
//                     transposed WY solve (nope_gdn_mlx.py:2637-2641, as block
//                     back substitution with the inverted diagonal blocks), the
//                     decay-masked K K^T / Q K^T products (nope_gdn_mlx.py:2080-2229,
//                     here through the anchored factors), the exponentials and
//                     the in-chunk reverse cumsum for dg (nope_gdn_mlx.py:2692-2693).
//                     Wave w owns dk-channel tile w: all per-(t, d) adjoints of
//                     that tile accumulate in its registers.
#include "kda_internal.h"

namespace kda {

// ----------------------------------------------------------------------------
// local adjoints
// ----------------------------------------------------------------------------

// rows of a (B, T, H, D) tensor as an A operand; rows at or past `valid` read as zero
template <typename TI>
__device__ __forceinline__ Fr8 frag8_rows(const TI* base, size_t rstride, int row0, int k0, int valid) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    Fr8 f;
    if (row0 + r < valid) {
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

// sum over the 16 lanes that share a lane group (same l/16)
__device__ __forceinline__ float sum16(float x) {
    x += __shfl_xor(x, 1, 64);
    x += __shfl_xor(x, 2, 64);
    x += __shfl_xor(x, 4, 64);
    x += __shfl_xor(x, 8, 64);
    return x;
}
// sum over the 4 lanes that share a column (same l%16)
__device__ __forceinline__ float sum4g(float x) {
    x += __shfl_xor(x, 16, 64);
    x += __shfl_xor(x, 32, 64);
    return x;
}

template <int D, typename TI, typename TG, int PREC>
__global__ __launch_bounds__(256) void kda_bwd_local_kernel(const LocalArgs a) {
    constexpr int NT = D / BS;
    __shared__ ChunkLds<D> s;
    __shared__ float sp[C][C + 4];           // Akk, then dP = diag(beta) dL
    __shared__ float sda[C][C + 4];          // dAqk
    __shared__ float sdr[C][2 * D + 4];      // dR = (I + L)^-T [dW | dU]
    __shared__ float tii[NB][BS][BS + 4];
    __shared__ float sdb[NB + NT][C];        // dbeta partials: [j] from dL tiles of column block j, [NB + nt] from channel tile nt

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    const int ch = blockIdx.x, bh = ch / a.nc, n = ch - bh * a.nc;
    const int b = bh / a.H, h = bh - b * a.H;
    const int t0 = n * C, valid = min(C, a.T - t0);
    const size_t rs = (size_t)a.H * D;
    const size_t base = ((size_t)b * a.T + t0) * rs + (size_t)h * D;
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

    // ---------------- phase 0: chunk factors, raw per-lane values ----------------
    for (int idx = tid; idx < C * C; idx += 256) sp[idx / C][idx % C] = a.Akk[cCC + idx];
    for (int idx = tid; idx < NB * BS * BS; idx += 256) {
        const int i = idx / (BS * BS), e = idx - i * BS * BS;
        tii[i][e / BS][e % BS] = a.Tii[(size_t)ch * NB * BS * BS + idx];
    }
    for (int idx = tid; idx < (NB + NT) * C; idx += 256) sdb[idx / C][idx % C] = 0.f;
    int flag = chunk_load<D, TI, TG>(s, q, k, g, beta, base, rs, bbase, a.H, valid);
    chunk_cumsum<D>(s);
    const int unsafe = chunk_factors<D, PREC>(s, flag);
    if (unsafe) chunk_band<D, 256>(s, __syncthreads_or(flag));

    // wave w owns channel tile nt = w: rows t = 16 m + 4 g4 + e, channel d
    const int nt = w;
    const bool own = nt < NT;
    const int d = own ? nt * BS + r16 : 0;
    float kx[NB][4], qx[NB][4], el[NB][4], er[NB][4], eb[NB][4], erb[NB];
    if (own) {
        const float G = s.g[C - 1][d];
#pragma unroll
        for (int m = 0; m < NB; ++m) {
            const float gr = s.g[BS * m][d];
            erb[m] = s.er[m][d];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                const float gt = s.g[t][d];
                kx[m][e] = s.kr[t][d];
                qx[m][e] = s.ql[t][d];
                el[m][e] = kexp<PREC>(gt - gr);
                er[m][e] = unsafe ? 0.f : kexp<PREC>(gr - gt);
                eb[m][e] = kexp<PREC>(G - gt);
            }
        }
    }
    __syncthreads();
    if (!unsafe) chunk_transform<D, PREC>(s, true);
    __syncthreads();
    // PHASE 1

    f32x4 dqa[NB], dka[NB], dga[NB], dWt[NB];
#pragma unroll
    for (int m = 0; m < NB; ++m) { dqa[m] = zero4(); dka[m] = zero4(); dga[m] = zero4(); dWt[m] = zero4(); }
    float dgcol = 0.f;

    // ---------------- phase 1: products over dv ----------------
    if (own) {
#pragma unroll
        for (int m = 0; m < NB; ++m) {
            f32x4 dQp = zero4(), dKb = zero4(), dW = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                const Fr8 Bh = frag8(hS, D, BS * nt, 32 * ks);
                const Fr8 Bdh = frag8(dhS, D, BS * nt, 32 * ks);
                dQp = mma8<PREC>(frag8_rows<TI>(dout + base, rs, BS * m, 32 * ks, valid), Bh, dQp);
                dKb = mma8<PREC>(frag8(Vp, D, BS * m, 32 * ks), Bdh, dKb);
                dW = mma8<PREC>(neg(frag8(dVp, D, BS * m, 32 * ks)), Bh, dW);
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
        // state-decay term of dG: e^G sum_col dh[d][col] h[d][col]
        float part = 0.f;
        for (int c = g4 * (D / 4); c < (g4 + 1) * (D / 4); ++c)
            part += ld1<TI>(dhS + (size_t)d * D + c) * ld1<TI>(hS + (size_t)d * D + c);
        dgcol = sum4g(dgcol) + kexp<PREC>(s.g[C - 1][d]) * sum4g(part);
    }
    // dAqk = tril(dO V'^T), 10 lower tiles over the 4 waves
    for (int tix = w; tix < 10; tix += 4) {
        int i, j;
        tile_ij(tix, i, j);
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks)
            acc = mma8<PREC>(frag8_rows<TI>(dout + base, rs, BS * i, 32 * ks, valid), frag8(Vp, D, BS * j, 32 * ks), acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
            sda[t][sx] = (sx <= t) ? acc[e] : 0.f;
        }
    }
    __syncthreads();

    // PHASE 2
    // ---------------- phase 2: transposed WY solve ----------------
    if (own) {
        f32x4 dRk[NB], dRv[NB];
#pragma unroll
        for (int i = NB - 1; i >= 0; --i) {
            f32x4 Yk = dWt[i], Yv;
#pragma unroll
            for (int e = 0; e < 4; ++e) Yv[e] = ld1<TI>(dVp + (size_t)(BS * i + 4 * g4 + e) * D + d);
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
        TI* dv = static_cast<TI*>(a.dv);
#pragma unroll
        for (int m = 0; m < NB; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                const float bt = s.beta[t];
                const float egt = erb[m] * el[m][e];
                const float vv = (t < valid) ? ld1<TI>(v + base + (size_t)t * rs + d) : 0.f;
                if (t < valid) st1<TI>(dv + base + (size_t)t * rs + d, bt * dRv[m][e]);
                dka[m][e] += bt * egt * dRk[m][e];
                dga[m][e] += dRk[m][e] * bt * egt * kx[m][e];
                const float db = sum16(dRv[m][e] * vv + dRk[m][e] * egt * kx[m][e]);
                if (r16 == 0) sdb[NB + nt][t] = db;
                sdr[t][d] = dRk[m][e];
                sdr[t][D + d] = dRv[m][e];
            }
        }
    }
    __syncthreads();

    // PHASE 3
    // ---------------- phase 3: dL = -tril(dR X^T, -1); dbeta; dP ----------------
    for (int tix = w; tix < 10; tix += 4) {
        int i, j;
        tile_ij(tix, i, j);
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2 * D / 32; ++ks) {
            const Fr8 A = frag8(&sdr[0][0], 2 * D + 4, BS * i, 32 * ks);
            const Fr8 B = (32 * ks < D) ? frag8(Wc, D, BS * j, 32 * ks) : frag8(Uc, D, BS * j, 32 * ks - D);
            acc = mma8<3>(A, B, acc);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
            const float dL = (sx < t) ? -acc[e] : 0.f;
            const float db = sum16(dL * sp[t][sx]);
            if (r16 == 0) sdb[j][t] = db;
            sp[t][sx] = s.beta[t] * dL;
        }
    }
    __syncthreads();

    // PHASE 4
    // ---------------- phase 4: decay-masked K K^T / Q K^T adjoints ----------------
    if (own) {
        if (!unsafe) {
            // row and column sides of a pair must agree to fp32 (see below): exact split products
            constexpr int PX = PREC >= 3 ? 4 : PREC;
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                f32x4 dKl = zero4(), dQl = zero4();
#pragma unroll
                for (int j = 0; j <= i; ++j) {
                    const float fs = (j < i) ? s.f[pair_idx(i, j)][d] : 1.f;
                    Fr4 B;
#pragma unroll
                    for (int e = 0; e < 4; ++e) B.v[e] = s.kr[BS * j + 4 * g4 + e][d] * fs;
                    dKl = mma4<PX>(frag4(&sp[0][0], C + 4, BS * i, BS * j), B, dKl);
                    Fr4 Aq = frag4(&sda[0][0], C + 4, BS * i, BS * j);
                    if (j == i) {   // the diagonal pairs (t, t) are added apart, below
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (4 * g4 + e == r16) Aq.v[e] = 0.f;
                    }
                    dQl = mma4<PX>(Aq, B, dQl);
                }
                Fr4 Bk, Bq;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    Bk.v[e] = s.kl[BS * i + 4 * g4 + e][d];
                    Bq.v[e] = s.ql[BS * i + 4 * g4 + e][d];
                }
                // The row-t and column-s contributions of each pair (t, s) to dgamma
                // cancel in the reverse cumsum below; weight each side by the very
                // operand values the other side's MFMA used (split to PREC), so that
                // the cancellation is exact to fp32 and the error stays independent
                // of the block's decay span.
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dka[i][e] += dKl[e] * el[i][e];
                    dqa[i][e] += dQl[e] * el[i][e];
                    dga[i][e] += dKl[e] * mfma_operand<PREC>(Bk.v[e]) + dQl[e] * mfma_operand<PREC>(Bq.v[e]);
                }
#pragma unroll
                for (int j = 0; j <= i; ++j) {
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
                        const float fac = fs * er[j][e];
                        dka[j][e] += dKr[e] * fac;
                        // the row side's B operand for this s and block pair
                        dga[j][e] -= dKr[e] * mfma_operand<PREC>(s.kr[BS * j + 4 * g4 + e][d] * fs);
                    }
                }
            }
        } else {
            // pairwise path: raw k in s.kr, raw q in s.ql, gamma in s.g
#pragma unroll
            for (int m = 0; m < NB; ++m) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * m + 4 * g4 + e;
                    const float gt = s.g[t][d];
                    float ak = 0.f, aq = 0.f, ag = 0.f;
                    // row t (dP[t][sx] strict, dA[t][sx]) and column t (dP[sx][t],
                    // dA[sx][t]) as two loops over the decay band
                    for (int sx = s.blo[t]; sx < t; ++sx) {
                        const float ks = s.kr[sx][d] * kexp<PREC>(gt - s.g[sx][d]);
                        const float pp = sp[t][sx], pa = sda[t][sx];
                        ak += pp * ks;
                        aq += pa * ks;
                        ag += (pp * kx[m][e] + pa * qx[m][e]) * ks;
                    }
                    for (int sx = t + 1; sx <= s.bhi[t]; ++sx) {
                        const float ex = kexp<PREC>(s.g[sx][d] - gt);
                        const float pp = sp[sx][t], pa = sda[sx][t];
                        const float c = (pp * s.kr[sx][d] + pa * s.ql[sx][d]) * ex;
                        ak += c;
                        ag -= c * kx[m][e];
                    }
                    dka[m][e] += ak;
                    dqa[m][e] += aq;
                    dga[m][e] += ag;
                }
            }
        }
        // The diagonal pairs (t, t) of A_qk (weight 1): dq_t += dA_tt k_t and
        // dk_t += dA_tt q_t, and nothing in dgamma_t, whose row and column terms
        // of such a pair are equal and opposite (summed into the two sides they
        // would dominate both, and the fp32 rounding of those sums would survive
        // the cancellation into dg).
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                dqa[m][e] += sda[t][t] * kx[m][e];
                dka[m][e] += sda[t][t] * qx[m][e];
            }

        // PHASE 5
        // ---------------- phase 5: dG, reverse cumsum, stores ----------------
        if (g4 == 3) dga[NB - 1][3] += dgcol;        // row C-1
        // suffix sums over rows t = 16 m + 4 g4 + e of this lane's channel
        float lsum[NB][4], tot[NB];
#pragma unroll
        for (int m = 0; m < NB; ++m) {
            float run = 0.f;
#pragma unroll
            for (int e = 3; e >= 0; --e) { run += dga[m][e]; lsum[m][e] = run; }
            tot[m] = run;
        }
        float after_m = 0.f;   // sum over row tiles > m
#pragma unroll
        for (int m = NB - 1; m >= 0; --m) {
            const float t0v = __shfl(tot[m], r16, 64);
            const float t1v = __shfl(tot[m], r16 + 16, 64);
            const float t2v = __shfl(tot[m], r16 + 32, 64);
            const float t3v = __shfl(tot[m], r16 + 48, 64);
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
                if (t < valid) {
                    const size_t o = base + (size_t)t * rs + d;
                    st1<TI>(dq + o, dqa[m][e]);
                    st1<TI>(dk + o, dka[m][e]);
                    st1<TG>(dg + o, lsum[m][e]);
                }
            }
    }
    if (tid < valid) {
        float db = 0.f;
#pragma unroll
        for (int j = 0; j < NB + NT; ++j) db += sdb[j][tid];
        st1<TI>(static_cast<TI*>(a.dbeta) + bbase + (size_t)tid * a.H, db);
    }
    // PHASE 6
}

// ----------------------------------------------------------------------------
// LDS plan of the bf16 local-adjoint kernel (kda_bwd_local3_kernel below;
// kda_bwd_local_kernel above serves fp32 inputs).
//
// Every global operand of the chunk arrives in one batch of 16-byte loads and
// lives in LDS; LDS regions are reused once their phase is over:
//   s          the chunk's q, k, gamma and anchored operands (ChunkSmem); the
//              g region later holds the solve's split A fragments and dL
//   region A   dO, V', h, dh (phase 1) -> dR (phases 2-3) -> dq/dk/dv/dg staging
//   region B   dV', v (phases 1-2)     -> dL when it does not fit in s.g (phases 3-4)
//   W, U       the chunk's WY factors (phases 1 and 3)
//   akk, tii   the recomputed A_kk and the inverted diagonal blocks of I + L
//   dA         dA_qk = tril(dO V'^T, -1) (phase 1 -> phase 4); its diagonal
//              is kept apart in pad column C (see phase 4)
// At D = 64, bf16: 155,648 bytes, one workgroup per CU.
// ----------------------------------------------------------------------------
template <int D, typename ST>
struct alignas(16) LocalSmem {
    static constexpr int PS = 16 / (int)sizeof(ST), LDK = D + PS, LDT = C + PS, LDA = C + 4, LDR = 2 * D + 4;
    ChunkSmem<D, ST> s;
    union {
        struct {
            ST dO[C][LDK];
            ST Vp[C][LDK];
            ST h[D][LDK];
            ST dh[D][LDK];
        } p1;
        float dR[C][LDR];
        ST out[4][C][LDK];
    } ra;
    union {
        struct {
            ST dVp[C][LDK];
            ST v[C][LDK];
        } p2;
        float dL[C][LDA];
    } rb;
    ST W[C][LDK];
    ST U[C][LDK];
    float akk[C][LDA];
    ST dA[C][LDT];
    float tii[NB][BS][BS + 4];
    float dbeta[C];
};

// The chunk's indices and its phase-0 tiles, handed from the kernel to its tail.
struct Local3Chunk {
    static constexpr int NPF = 1;   // prefetch lines per thread
    int tid, w, l, r16, g4, ct, rh, valid;
    size_t rs, base, bbase;
    const char* pf[NPF];            // the thread's prefetch line addresses, or null
};
template <int D, typename ST>
struct Local3Tiles {
    Tile<ST, C, D, 512> W, U, dO, v, dVp;
    Tile<ST, D, D, 512> h, dh;
};

// ----------------------------------------------------------------------------
// local adjoints, bf16 operands, 8 waves (two per SIMD, so each hides the
// other's latencies).  Wave w owns channel tile ct = w % 4 and row half
// rh = w / 4 (row blocks 2 rh, 2 rh + 1) of every per-(t, d) adjoint.
//   phase 1  dQp, dKb, dW of the own rows; dA tiles over all waves
//   phase 2  the transposed solve splits by right-hand side: the rh = 0 waves
//            run the dW chain, the rh = 1 waves the dV' chain, each for its
//            channel tile, through LDS (dR)
//   phase 3  dL tiles over all waves; dbeta row sums
//   phase 4  decay-masked adjoints: every wave computes exactly the
//            contributions to its own rows (row blocks i of dK_l / dQ_l, and
//            row blocks j of dK_r)
//   phase 5  in-chunk reverse cumsum of dgamma: the two row halves meet
//            through one LDS total per channel
// A_kk, its diagonal-block inverses and V' = U - W h are recomputed here from
// what is already in LDS instead of being read from the workspace.
// LDS regions and their reuse: the plan above LocalSmem.
// ----------------------------------------------------------------------------
template <int D, typename ST, typename TG, int PREC, bool STRONG>
__device__ __forceinline__ void local3_tail(const LocalArgs& a, LocalSmem<D, ST>& sm, float* xg, float* xt,
                                            char* pfbuf, const Local3Chunk& c, Local3Tiles<D, ST>& tl, float braw,
                                            int dfl) {
    using L = LocalSmem<D, ST>;
    constexpr int NTH = 512, NT = D / BS, LDK = L::LDK, LDT = L::LDT, LDA = L::LDA, LDR = L::LDR;
    auto& s = sm.s;
    const int tid = c.tid, w = c.w, l = c.l, r16 = c.r16, g4 = c.g4, ct = c.ct, rh = c.rh, valid = c.valid;
    __builtin_assume(w >= 0 && w < 8);
    const size_t rs = c.rs, base = c.base, bbase = c.bbase;
    auto &tW = tl.W, &tU = tl.U, &tdo = tl.dO, &tv = tl.v, &tdVp = tl.dVp;
    auto &th = tl.h, &tdh = tl.dh;
    const bool unsafe = STRONG && (dfl & 16) != 0;           // g > 0 or NaN: every pair pairwise
    const int pmask = (STRONG && !unsafe) ? (dfl & 15) : 0;  // diagonal blocks beyond the span guard
    if (tid < C) s.beta[tid] = (tid < valid) ? braw : 0.f;
    tW.store(&sm.W[0][0], LDK);
    tU.store(&sm.U[0][0], LDK);
    th.store(&sm.ra.p1.h[0][0], LDK);

    // per-lane values of the owned (t, d): rows t = 16 m + 4 g4 + e, m = 2 rh + mm, channel d
    const bool own = ct < NT;
    const int d = own ? ct * BS + r16 : 0;
    constexpr int MB = NB / 2;
    // el = e^{a_t}, er = e^{b_t} (the anchored operand factors), eb = e^{G - gamma_t},
    // erb = e^{gamma_{16m-1}}, so e^{gamma_t} = erb el; at = a_t and fdm = e^{-T_m}
    // serve the pairwise diagonal tiles and the diagonal tile factor of phase 4
    float kx[MB][4], qx[MB][4], el[MB][4], er[MB][4], eb[MB][4], at[MB][4], erb[MB], fdm[MB], eGd;
    {
        const float Tb[NB] = {s.g[BS - 1][d], s.g[2 * BS - 1][d], s.g[3 * BS - 1][d], s.g[4 * BS - 1][d]};
        eGd = kexp<PREC>((Tb[0] + Tb[1]) + (Tb[2] + Tb[3]));
#pragma unroll
        for (int mm = 0; mm < MB; ++mm) {
            const int m = 2 * rh + mm;
            erb[mm] = fac_ep(s, m, d);
            fdm[mm] = s.fac[FAC_FD + m][d];
            float sfx = 0.f;   // G - gamma_{16m+15}
#pragma unroll
            for (int mq = m + 1; mq < NB; ++mq) sfx += Tb[mq];
            const float eqm = fac_eq(s, m, d);
            // raw k and q of the lane's rows, column d (transposing reads)
            ld_col4(&s.kr[0][0], LDK, BS * ct, BS * m, kx[mm]);
            ld_col4(&s.ql[0][0], LDK, BS * ct, BS * m, qx[mm]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * m + 4 * g4 + e;
                const float a_t = s.g[t][d], b_t = Tb[m] - a_t;
                at[mm][e] = a_t;
                el[mm][e] = kexp<PREC>(a_t);
                er[mm][e] = unsafe ? 0.f : kexp<PREC>(b_t);
                eb[mm][e] = unsafe ? kexp<PREC>(b_t + sfx) : er[mm][e] * eqm;
            }
        }
    }
    // Diagonal tiles of the blocks in pmask, from raw k (before the transform
    // overwrites it): wave w < 4 forms block w's tile with 4-row sub-anchors on
    // MFMA; blocks in qmask (4-row sub-blocks beyond the guard too) pair by
    // pair, A_kk[t][s] = sum_d k_t k_s e^{a_t - a_s}, one tile entry per thread
    // and step.  The other tiles are formed by MFMA below.
    const int qmask = pmask & (dfl >> 5);
    // With two k-steps (D = 64) waves w and w + 4 share block w's sub-anchored
    // tile, a channel half each: the second half's partial product waits in the
    // dA tile (dead until phase 1) and wave w adds it before inverting the block.
    constexpr bool SUBSPLIT = D / 32 == 2;
    float (*sub2)[BS][BS] = reinterpret_cast<float (*)[BS][BS]>(&sm.dA[0][0]);
    static_assert(!SUBSPLIT || sizeof(sm.dA) >= sizeof(float) * NB * BS * BS, "second halves fit the dA tile");
    if (pmask) {
        const int blk = SUBSPLIT ? (w & (NB - 1)) : w, half = SUBSPLIT ? (w >> 2) : 0;
        if ((SUBSPLIT || w < NB) && (((pmask & ~qmask) >> blk) & 1)) {
            f32x4 P, Q;
            subanchor_tile<D, ST, PREC, false>(s, blk, P, Q, SUBSPLIT ? half : -1);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * blk + 4 * g4 + e, sx = BS * blk + r16;
                if (half == 0) sm.akk[t][sx] = (sx < t) ? P[e] : 0.f;
                else sub2[blk][4 * g4 + e][r16] = P[e];
            }
        }
        const int nent = __popc(qmask) * BS * BS;
        for (int pp = tid; pp < nent; pp += NTH) {
            const int kb = pp / (BS * BS), e = pp - kb * BS * BS;
            int blk = 0;
            for (int mq = qmask, c = 0;; mq &= mq - 1, ++c)
                if (c == kb) { blk = __ffs(mq) - 1; break; }
            const int t = BS * blk + e / BS, sx = BS * blk + e % BS;
            float ak = 0.f;
            if (sx < t)
#pragma unroll 2
                for (int dd = 0; dd < D; ++dd)
                    ak += ld1<ST>(&s.kr[t][dd]) * (ld1<ST>(&s.kr[sx][dd]) * kexp<PREC>(s.g[t][dd] - s.g[sx][dd]));
            sm.akk[t][sx] = ak;
        }
    }
    __syncthreads();
    if (!unsafe) {
        // K_l = K e^{a}, Q_l = Q e^{a}, K_r = K e^{b}, b = T_blk - a
        constexpr int EPV = 16 / (int)sizeof(ST), VPR = D / EPV;
        for (int vv = tid; vv < C * VPR; vv += NTH) {
            const int t = vv / VPR, c0 = (vv - t * VPR) * EPV, te = (t & ~(BS - 1)) + BS - 1;
            const Vec16<ST> qv{*reinterpret_cast<const uint4*>(&s.ql[t][c0])};
            const Vec16<ST> kv{*reinterpret_cast<const uint4*>(&s.kr[t][c0])};
            float okl[EPV], oql[EPV], okr[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float x = s.g[t][c0 + e];
                const float e1 = kexp<PREC>(x), e2 = kexp<PREC>(s.g[te][c0 + e] - x);
                okl[e] = kv.get(e) * e1;
                oql[e] = qv.get(e) * e1;
                okr[e] = kv.get(e) * e2;
            }
            store_vec<ST>(&s.kl[t][c0], okl);
            store_vec<ST>(&s.ql[t][c0], oql);
            store_vec<ST>(&s.kr[t][c0], okr);
        }
    }
    tdo.store(&sm.ra.p1.dO[0][0], LDK);
    tv.store(&sm.rb.p2.v[0][0], LDK);
    tdVp.store(&sm.rb.p2.dVp[0][0], LDK);
    tdh.store(&sm.ra.p1.dh[0][0], LDK);
    __syncthreads();

    // Split A fragments of the phase-2 solve, written once by the waves that form
    // A_kk and the inverses (anchored path), read by every solving wave with one
    // 16-byte read per lane: fc[64 i + lane] = T_ii^T, fc[64 (4 + p) + lane] =
    // A_ij = -L_ji^T for pair p = (j, i), j > i.  They live in the g region, dead
    // on this path from here until dL takes it in phase 3 (D >= 64: at D = 32
    // the region is too small and the solve reads A_kk and the inverses).
    constexpr bool FC = 10 * 64 * sizeof(Frag4) <= sizeof(s.g);
    Frag4* fc = reinterpret_cast<Frag4*>(&s.g[0][0]);

    // ---------------- recomputed intermediates ----------------
    // A_kk = strict-lower(K K^T . decay), formed as the prep kernel forms it, its
    // diagonal-block inverses, and V' = U - W h (h is the chunk-start state in the
    // bf16 the state recurrence used, so V' equals what it computed).  Waves 0-3
    // each form one diagonal tile of A_kk and invert it at once (their own LDS
    // writes, no barrier); waves 4-7 form the off-diagonal tiles; V' is split
    // over all eight waves.
    auto akk_tile = [&](int i, int j) __attribute__((always_inline)) {
        // B operand: K_r of block j times the tile's channel factor (F_ij, 1
        // between adjacent blocks, e^{-T_i} on the diagonal), as prep forms it
        const float* fsc = &s.fac[(j == i) ? FAC_FD + i : (j == i - 1) ? 0 : fac_f_row(i, j)][0];
        f32x4 P = zero4();
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const Frag8 Ak = ldfrag_c<PREC, ST>(&s.kl[0][0], LDK, BS * i, 32 * ks);
            const Frag8 Bk = (j == i - 1) ? ldfrag_c<PREC, ST>(&s.kr[0][0], LDK, BS * j, 32 * ks)
                                          : ldfrag_c_scaled<PREC, ST>(&s.kr[0][0], LDK, BS * j, 32 * ks, fsc + 32 * ks);
            P = mma<PREC>(Ak, Bk, P);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
            sm.akk[t][sx] = (sx < t) ? P[e] : 0.f;
        }
        if (FC && j < i) {
            // this lane's P[e] = A_kk[16i + 4 g4 + e][16j + r16] is exactly what the
            // same lane of A_ji = -L_ij^T holds: A[r16][4 g4 + e]
            float lv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) lv[e] = -s.beta[BS * i + 4 * g4 + e] * P[e];
            fc[64 * (4 + pair_idx(i, j)) + l] = frag4_from_f32<3>(lv);
        }
    };
    auto vp_tile = [&](int tix) __attribute__((always_inline)) {
        const ST* sh = &sm.ra.p1.h[0][0];
        const int m = tix / NT, c = tix - m * NT;
        f32x4 P = zero4();
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const Frag8 A = ldfrag<PREC, ST>(&sm.W[0][0], LDK, BS * m, 32 * ks);
            // B[k][n] = h[k][n]: h is stored with k along its rows, read transposed
            P = mma<PREC>(A, ldfragT(sh, LDK, BS * c, 32 * ks), P);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * m + 4 * g4 + e, cc = BS * c + r16;
            st1<ST>(&sm.ra.p1.Vp[t][cc], ld1<ST>(&sm.U[t][cc]) - P[e]);
        }
    };
    if (!unsafe) {
        if (w < NB) {
            // a diagonal tile of pmask was formed before the transform (sub-anchored:
            // its second channel half is added here)
            if (!((pmask >> w) & 1)) {
                akk_tile(w, w);
            } else if (SUBSPLIT && !((qmask >> w) & 1)) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * w + 4 * g4 + e, sx = BS * w + r16;
                    if (sx < t) sm.akk[t][sx] += sub2[w][4 * g4 + e][r16];
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave reads back its own tile
            diag_inverse_reg<LDA>(&sm.akk[0][0], s.beta, sm.tii, FC ? fc : nullptr);
        } else {
            constexpr int OFF[6] = {1, 3, 4, 6, 7, 8};   // tile_ij indices of the blocks below the diagonal
            for (int o = w - NB; o < 6; o += 8 - NB) {
                int i, j;
                tile_ij(OFF[o], i, j);
                akk_tile(i, j);
            }
        }
        for (int idx = tid; idx < 6 * BS * BS; idx += NTH) {
            const int tile = idx / (BS * BS), e = idx - tile * BS * BS;
            const int i = (tile < 3) ? 0 : (tile < 5) ? 1 : 2;
            const int j = (tile < 3) ? tile + 1 : (tile < 5) ? tile - 1 : 3;
            sm.akk[BS * i + e / BS][BS * j + (e % BS)] = 0.f;
        }
    } else {
        // every pair pairwise (g > 0 or NaN in the chunk): raw k in kr, exact
        // exp(gamma_t - gamma_s)
        for (int p = tid; p < C * C; p += NTH) {
            const int t = p / C, sx = p - t * C;
            float ak = 0.f;
            if (sx < t)
#pragma unroll 1
                for (int dd = 0; dd < D; ++dd)
                    ak += ld1<ST>(&s.kr[t][dd]) *
                          (ld1<ST>(&s.kr[sx][dd]) * kexp<PREC>(chunk_gamma(s, t, dd) - chunk_gamma(s, sx, dd)));
            sm.akk[t][sx] = ak;
        }
        __syncthreads();
        if (w < NB) diag_inverse_reg<LDA>(&sm.akk[0][0], s.beta, sm.tii);
    }
    // V' tiles by measured finish times of the work above: waves 0-3 (a
    // diagonal tile and its inverse) take two each, waves 4-5 (two
    // off-diagonal tiles) one, waves 6-7 (one off-diagonal tile) three
    static_assert(NB == 4, "wave roles assume four row blocks");
    {
        const int v0 = (w < 4) ? 2 * w : (w < 6) ? w + 4 : 3 * w - 8;   // 0 2 4 6 | 8 9 | 10 13
        const int vn = (w < 4) ? 2 : (w < 6) ? 1 : 3;
        for (int i = 0; i < vn; ++i) {
            const int tix = v0 + i;
            if (tix < NB * NT) vp_tile(tix);
        }
    }
    __syncthreads();

    // L2 prefetch of the chunk this XCD starts next: its line addresses were
    // formed by the kernel (Local3Chunk::pf).  The landing bytes are scratch.
    {
        const uint32_t m = lds_addr(pfbuf);
#pragma unroll
        for (int i = 0; i < Local3Chunk::NPF; ++i)
            if (c.pf[i] != nullptr) dma4(c.pf[i], m);
    }
    f32x4 dqa[MB], dka[MB], dga[MB], dWt[NB];
    float dgcol = 0.f, part = 0.f;

    // Operands of the phase-2 solve, read now so that their LDS latency hides
    // behind phase 1: T_ii^T and A_ij = -L_ji^T blocks, and (rh = 1) Y = dV'.
    f32x4 Y[NB];
    Frag4 At[NB], Aij[6];
    if (own) {
        if (rh) {
            // column d of dV', rows 16 i + 4 g4 + e (transposing reads)
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                float yv[4];
                ld_col4(&sm.rb.p2.dVp[0][0], LDK, BS * ct, BS * i, yv);
                Y[i] = f32x4{yv[0], yv[1], yv[2], yv[3]};
            }
        }
        if (FC && !unsafe) {
#pragma unroll
            for (int i = 0; i < NB; ++i) At[i] = fc[64 * i + l];
#pragma unroll
            for (int p = 0; p < 6; ++p) Aij[p] = fc[64 * (4 + p) + l];
        } else {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                float tv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) tv[e] = sm.tii[i][4 * g4 + e][r16];     // A[a][b] = T_ii[b][a]
                At[i] = frag4_from_f32<3>(tv);
            }
#pragma unroll
            for (int j = 1; j < NB; ++j)
#pragma unroll
                for (int i = 0; i < j; ++i) {
                    float av[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int rb = BS * j + 4 * g4 + e;
                        av[e] = -s.beta[rb] * sm.akk[rb][BS * i + r16];
                    }
                    Aij[pair_idx(j, i)] = frag4_from_f32<3>(av);
                }
        }
    }

    // ---------------- phase 1: products over dv ----------------
    {
        const ST* sdO = &sm.ra.p1.dO[0][0];
        const ST* sVp = &sm.ra.p1.Vp[0][0];
        const ST* sdVp = &sm.rb.p2.dVp[0][0];
        const ST* sh = &sm.ra.p1.h[0][0];
        const ST* sdh = &sm.ra.p1.dh[0][0];
        if (own) {
            Frag8 Ao[MB][D / 32], Av[MB][D / 32], Bh[D / 32], Bdh[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                // every phase-1 product takes both operands from LDS rows:
                // contiguous k-slots (ldfrag_c), one 16-byte read per operand
                Bh[ks] = ldfrag_c<PREC, ST>(sh, LDK, BS * ct, 32 * ks);
                Bdh[ks] = ldfrag_c<PREC, ST>(sdh, LDK, BS * ct, 32 * ks);
#pragma unroll
                for (int mm = 0; mm < MB; ++mm) {
                    const int m = 2 * rh + mm;
                    Ao[mm][ks] = ldfrag_c<PREC, ST>(sdO, LDK, BS * m, 32 * ks);
                    Av[mm][ks] = ldfrag_c<PREC, ST>(sVp, LDK, BS * m, 32 * ks);
                }
            }
            // dW = -dV' h^T, all row blocks of the channel tile, for the rh = 0
            // waves, which run the dW chain of the solve from registers
            if (rh == 0) {
#pragma unroll
                for (int m = 0; m < NB; ++m) {
                    f32x4 dW = zero4();
#pragma unroll
                    for (int ks = 0; ks < D / 32; ++ks)
                        dW = mma<PREC>(ldfrag_c<PREC, ST>(sdVp, LDK, BS * m, 32 * ks), Bh[ks], dW);
                    dWt[m] = negacc(dW);
                }
            }
            // state-decay term of dG (rh = 0 waves, which have the shorter phase 1):
            // e^G sum_col dh[d][col] h[d][col], lane (g4, d) over columns
            // 16 g4 .. 16 g4 + 15 in 16-byte reads
            if (rh == 0) {
#pragma unroll
                for (int c8 = 0; c8 < D / 4; c8 += 8) {
                    const int cc = g4 * (D / 4) + c8;
                    const Vec16<ST> x{*reinterpret_cast<const uint4*>(sdh + d * LDK + cc)};
                    const Vec16<ST> y{*reinterpret_cast<const uint4*>(sh + d * LDK + cc)};
#pragma unroll
                    for (int e = 0; e < 8; ++e) part += x.get(e) * y.get(e);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mm = 0; mm < MB; ++mm) {
                f32x4 dQp = zero4(), dKb = zero4();
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    dQp = mma<PREC>(Ao[mm][ks], Bh[ks], dQp);
                    dKb = mma<PREC>(Av[mm][ks], Bdh[ks], dKb);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float egt = erb[mm] * el[mm][e];                // e^{gamma_t}
                    const float kbv = kx[mm][e] * eb[mm][e];              // Kb
                    dqa[mm][e] = dQp[e] * egt;
                    dka[mm][e] = dKb[e] * eb[mm][e];
                    dga[mm][e] = dQp[e] * qx[mm][e] * egt - dKb[e] * kbv;
                    dgcol += dKb[e] * kbv;
                }
            }
            dgcol = sum4g(dgcol);
            part = sum4g(part);
            if (rh == 0 && g4 == 0) xg[d] = dgcol + eGd * part;
        }
        // dAqk = tril(dO V'^T): 10 lower tiles over the 8 waves, one each and the
        // last two for waves 4-5 (the rh = 1 waves end phase 1 before the rh = 0
        // waves, which also form dW)
        for (int tix = (w < 4) ? w + 4 : w - 4; tix < 10; tix += (w < 4) ? 10 : 8) {
            int i, j;
            tile_ij(tix, i, j);
            Frag8 A[D / 32], B[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                A[ks] = ldfrag_c<PREC, ST>(sdO, LDK, BS * i, 32 * ks);
                B[ks] = ldfrag_c<PREC, ST>(sVp, LDK, BS * j, 32 * ks);
            }
            f32x4 acc = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) acc = mma<PREC>(A[ks], B[ks], acc);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
                st1<ST>(&sm.dA[t][sx], (sx < t) ? acc[e] : 0.f);
                if (sx == t) st1<ST>(&sm.dA[t][C], acc[e]);   // the diagonal, in the pad column
            }
        }
    }

    // ---------------- phase 2: transposed WY solve, by right-hand side ----------------
    // Each wave goes on from its own phase 1 (the operands are in registers or
    // unchanged LDS); dR reaches region A only after the barrier that ends phase 1.
    f32x4 X[NB];
    if (own) {
        // rh = 0: Y = dW (registers), result dR[:, d]; rh = 1: Y = dV', result dR[:, D + d].
        // Right-looking block back substitution: as soon as dR_j is known, every
        // earlier block is updated, Y_i += A_ij dR_j with
        // A_ij[a][b] = -L[16j + b][16i + a] = -beta_{16j+b} Akk[16j+b][16i+a].
        if (!rh) {
#pragma unroll
            for (int i = 0; i < NB; ++i) Y[i] = dWt[i];
        }
#pragma unroll
        for (int j = NB - 1; j >= 0; --j) {
            X[j] = mma4f<3>(At[j], accfrag4<3>(Y[j]), zero4());
            const Frag4 Bj = accfrag4<3>(X[j]);
#pragma unroll
            for (int i = 0; i < j; ++i) Y[i] = mma4f<3>(Aij[pair_idx(j, i)], Bj, Y[i]);
        }
    }
    __syncthreads();   // phase-1 operands (region A) are dead from here
    if (own) {
        const int col = rh ? D + d : d;
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) sm.ra.dR[BS * j + 4 * g4 + e][col] = X[j][e];
    }
    __syncthreads();
    // contributions of dR to the own rows; dv = beta dR_v
    f32x4 dvo[MB];
    if (own) {
#pragma unroll
        for (int mm = 0; mm < MB; ++mm)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * (2 * rh + mm) + 4 * g4 + e;
                const float bt = s.beta[t], egt = erb[mm] * el[mm][e];
                const float rk = sm.ra.dR[t][d];
                dka[mm][e] += bt * egt * rk;
                dga[mm][e] += rk * bt * egt * kx[mm][e];
                dvo[mm][e] = bt * sm.ra.dR[t][D + d];
            }
    }
    // dbeta, part 1: sum_d dV~[t][d] v[t][d] + dK~[t][d] e^{gamma_t} k[t][d]; 8 threads per row,
    // each over D / 8 consecutive channels (vector reads; a wave's rows share one block)
    {
        const int t = tid >> 3, qd = tid & 7, d0 = qd * (D / 8);
        float acc = 0.f;
        if (!unsafe) {
            const float* fe = (t >= BS) ? &s.fac[FAC_EP + t / BS - 1][d0] : nullptr;
#pragma unroll
            for (int c4 = 0; c4 < D / 8; c4 += 4) {
                const float4 rv = *reinterpret_cast<const float4*>(&sm.ra.dR[t][D + d0 + c4]);
                const float4 rk = *reinterpret_cast<const float4*>(&sm.ra.dR[t][d0 + c4]);
                const float4 vv = ld4<ST>(&sm.rb.p2.v[t][d0 + c4]);
                float4 kv = ld4<ST>(&s.kl[t][d0 + c4]);
                if (fe) {
                    const float4 f = *reinterpret_cast<const float4*>(fe + c4);
                    kv = make_float4(kv.x * f.x, kv.y * f.y, kv.z * f.z, kv.w * f.w);
                }
                acc += rv.x * vv.x + rk.x * kv.x;
                acc += rv.y * vv.y + rk.y * kv.y;
                acc += rv.z * vv.z + rk.z * kv.z;
                acc += rv.w * vv.w + rk.w * kv.w;
            }
        } else {
            for (int dd = d0; dd < d0 + D / 8; ++dd) {
                const float egk = ld1<ST>(&s.kr[t][dd]) * kexp<PREC>(chunk_gamma(s, t, dd));
                acc += sm.ra.dR[t][D + dd] * ld1<ST>(&sm.rb.p2.v[t][dd]) + sm.ra.dR[t][dd] * egk;
            }
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        acc += __shfl_xor(acc, 4, 64);
        if (qd == 0) sm.dbeta[t] = acc;
    }
    // dL goes to the g region, dead on the anchored path, when it fits (D >= 64):
    // then phase 3 need not wait for the v reads above.  Otherwise it reuses
    // region B once v and dV' are dead.
    constexpr int LDG = ChunkSmem<D, ST>::LDG;
    constexpr bool DL_IN_G = LDG >= LDA;
    const bool dl_g = DL_IN_G && !unsafe;
    float* sdL = dl_g ? &s.g[0][0] : &sm.rb.dL[0][0];
    constexpr int LDL = DL_IN_G ? LDG : LDA;
    static_assert(!DL_IN_G || LDG == LDA, "one dL stride");
    if (!dl_g) __syncthreads();   // v and dV' (region B) are dead from here
    // With dL in the g region, the bf16 P = beta_t dL[t][s] -- the A operand of
    // phase 4's row and column sides, as both round it -- also goes to the dV'
    // tile of region B (dead since phase 1), so that phase 4 reads it as
    // fragments: rows by row reads, columns by transposing reads.
    constexpr bool PB = DL_IN_G && L::LDK >= C + 8;
    const bool pb = PB && dl_g;
    ST* sP = &sm.rb.p2.dVp[0][0];

    // ---------------- phase 3: dL = -tril(dR X^T, -1) ----------------
    for (int tix = w; tix < 10; tix += 8) {
        int i, j;
        tile_ij(tix, i, j);
        Frag8 A[2 * D / 32], B[2 * D / 32];
#pragma unroll
        for (int ks = 0; ks < 2 * D / 32; ++ks) {
            A[ks] = ldfrag_c<2, float>(&sm.ra.dR[0][0], LDR, BS * i, 32 * ks);
            B[ks] = (32 * ks < D) ? ldfrag_c<1, ST>(&sm.W[0][0], LDK, BS * j, 32 * ks)
                                  : ldfrag_c<1, ST>(&sm.U[0][0], LDK, BS * j, 32 * ks - D);
        }
        // W and U are bf16 here: splitting only dR keeps the fp32 accuracy of the product
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < 2 * D / 32; ++ks) acc = mma<2>(A[ks], B[ks], acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
            const float v = (sx < t) ? -acc[e] : 0.f;
            sdL[t * LDL + sx] = v;
            if (pb) st1<ST>(sP + t * LDK + sx, s.beta[t] * v);
        }
    }
    __syncthreads();
    // dbeta, part 2: sum_s dL[t][s] Akk[t][s]
    {
        const int t = tid >> 3, qd = tid & 7;
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < C / 8; ++c) {
            const int sx = qd * (C / 8) + c;
            acc += sdL[t * LDL + sx] * sm.akk[t][sx];
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        acc += __shfl_xor(acc, 4, 64);
        if (qd == 0) sm.dbeta[t] += acc;
    }

    // ---------------- phase 4: decay-masked K K^T / Q K^T adjoints, own rows ----------------
    if (own) {
        if (!unsafe) {
            // The tile factor (F_ij between blocks, e^{-T_i} on the diagonal) is per
            // channel, so it scales the accumulated product instead of the B operand.
            // Diagonal tiles of blocks in pmask are evaluated pair by pair below.
            auto colfrag = [&](const ST* M, int ld, int row0) __attribute__((always_inline)) {
                // B[k][n] = M[row0 + k][d] for the lane's k = 4 g4 + 0..3, raw bf16
                return ldfrag4T_tr(M, ld, BS * ct, row0);
            };
#pragma unroll
            for (int mm = 0; mm < MB; ++mm) {
                const int i = 2 * rh + mm;
                // rows of block i: dK_l = sum_{j <= i} F_ij dP[i][j] K_r[j], dQ_l likewise with dA
                const float bi = s.beta[BS * i + r16];
                f32x4 dKl = zero4(), dQl = zero4();
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    if (j > i || (j == i && ((pmask >> i) & 1))) continue;
                    const Frag4 B = colfrag(&s.kr[0][0], LDK, BS * j);
                    Frag4 Ap;
                    if (pb) {
                        Ap = ldfrag4<1, ST>(sP, LDK, BS * i, BS * j);
                    } else {
                        const float4 x = *reinterpret_cast<const float4*>(sdL + (BS * i + r16) * LDL + BS * j + 4 * g4);
                        const float pv[4] = {bi * x.x, bi * x.y, bi * x.z, bi * x.w};
                        Ap = frag4_from_f32<1>(pv);
                    }
                    const f32x4 Pk = mma4f<1>(Ap, B, zero4());
                    // dA is strictly lower: the diagonal pairs (t, t) are added apart, below
                    const Frag4 Aq = ldfrag4<1, ST>(&sm.dA[0][0], LDT, BS * i, BS * j);
                    const f32x4 Pq = mma4f<1>(Aq, B, zero4());
                    const float fs = (j < i) ? fac_tile(s, i, j, d) : fdm[mm];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dKl[e] += Pk[e] * fs;
                        dQl[e] += Pq[e] * fs;
                    }
                }
                // dgamma: weight by the bf16 values the column side's MFMAs read
                // (K_l, Q_l of row t) so that each pair cancels exactly in the
                // reverse cumsum, whatever the decay span
                float klv[4], qlv[4];
                ld_col4(&s.kl[0][0], LDK, BS * ct, BS * i, klv);
                ld_col4(&s.ql[0][0], LDK, BS * ct, BS * i, qlv);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dka[mm][e] += dKl[e] * el[mm][e];
                    dqa[mm][e] += dQl[e] * el[mm][e];
                    dga[mm][e] += dKl[e] * klv[e] + dQl[e] * qlv[e];
                }
            }
#pragma unroll
            for (int mm = 0; mm < MB; ++mm) {
                const int j = 2 * rh + mm;
                // rows of block j: dK_r = sum_{i >= j} F_ij (dP[i][j]^T K_l[i] + dA[i][j]^T Q_l[i]),
                // then times e^{b}
                f32x4 dKr = zero4();
#pragma unroll
                for (int i = 0; i < NB; ++i) {
                    if (i < j || (i == j && ((pmask >> j) & 1))) continue;
                    Frag4 Ap, Aa;   // dP^T, dA^T: rows s = 16 j + r16, k = t = 16 i + 4 g4 + e
                    if (pb) {
                        Ap = ldfrag4T_tr(sP, LDK, BS * j, BS * i);
                        Aa = ldfrag4T_tr(&sm.dA[0][0], LDT, BS * j, BS * i);
                    } else {
                        float pv[4], av[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int t = BS * i + 4 * g4 + e;
                            pv[e] = s.beta[t] * sdL[t * LDL + BS * j + r16];
                            av[e] = ld1<ST>(&sm.dA[t][BS * j + r16]);
                        }
                        Ap = frag4_from_f32<1>(pv);
                        Aa = frag4_from_f32<1>(av);
                    }
                    f32x4 P = mma4f<1>(Ap, colfrag(&s.kl[0][0], LDK, BS * i), zero4());
                    P = mma4f<1>(Aa, colfrag(&s.ql[0][0], LDK, BS * i), P);
                    const float fs = (j < i) ? fac_tile(s, i, j, d) : fdm[mm];
#pragma unroll
                    for (int e = 0; e < 4; ++e) dKr[e] += P[e] * fs;
                }
                float krv[4];   // the row side's B operand (K_r of row s, raw bf16)
                ld_col4(&s.kr[0][0], LDK, BS * ct, BS * j, krv);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dka[mm][e] += dKr[e] * er[mm][e];
                    dga[mm][e] -= dKr[e] * krv[e];
                }
            }
            // Diagonal tiles of own blocks in pmask & ~qmask, with the 4-row
            // sub-anchors of subanchor_tile: pair (t, s), t in sub-block p, s in
            // sub-block q <= p, splits as e^{a_t - a_{r_p}} * e^{a_{r_p} - a_s}.
            // Everything comes from the lane's own rows (row 16 m + 4 g + e of
            // channel d is register e of lane (g, d)), plus the anchors a_{r_p},
            // rows 4 p - 1 of the block, from lanes (p - 1, d).
            //   A_t = bf16(K_t e^{a_t - a_{r_g}}), Aq_t likewise with Q: the row
            //     factor of the lane's rows;
            //   B^p_s = bf16(K_s e^{a_{r_p} - a_s}) for p >= g (0 for p < g).
            // Row side, pass p: rows t of sub-block p (dP / dA masked to them)
            // against B^p; a lane's rows come from pass p = g.  Column side, pass
            // p: dP^T / dA^T against A / Aq of rows t in sub-block p (the lanes
            // g == p), combined with B^p of the lane's own rows.  Each pair's two
            // dgamma terms multiply the same bf16 A_t and B^p_s, so they cancel
            // exactly in the reverse cumsum.
#pragma unroll
            for (int mm = 0; mm < MB; ++mm) {
                const int m = 2 * rh + mm;
                if (!(((pmask & ~qmask) >> m) & 1)) continue;
                float arp[NB];
                arp[0] = 0.f;
#pragma unroll
                for (int p = 1; p < NB; ++p) arp[p] = __shfl(at[mm][3], 16 * (p - 1) + r16, 64);
                const float arg = (g4 == 0) ? arp[0] : (g4 == 1) ? arp[1] : (g4 == 2) ? arp[2] : arp[3];
                // Pass factors e^{a_{r_p} - a_t} (p >= g, 0 before) as W_p V_t, with
                // a_l the lane's last row l = 16 m + 4 g + 3: W_p = e^{a_{r_p} - a_l}
                // (<= e^{4-row span} for p = g, <= 1 after), V_t = e^{a_l - a_t} in
                // [e^{-4-row span}, 1].  Neither factor overflows; where W_p underflows
                // the product is below it.  (A large negative exponent gives W_p = 0
                // for p < g: no per-element select.)
                float eo[4], vt[4], wp[NB];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    eo[e] = kexp<PREC>(at[mm][e] - arg);
                    vt[e] = (e == 3) ? 1.f : kexp<PREC>(at[mm][3] - at[mm][e]);
                }
#pragma unroll
                for (int p = 0; p < NB; ++p) wp[p] = kexp<PREC>(((p >= g4) ? arp[p] : -1e30f) - at[mm][3]);
                // A_t, Aq_t as packed bf16 pairs, and the same values back as floats
                const uint32_t ak0 = pack2bf(kx[mm][0] * eo[0], kx[mm][1] * eo[1]);
                const uint32_t ak1 = pack2bf(kx[mm][2] * eo[2], kx[mm][3] * eo[3]);
                const uint32_t aq0 = pack2bf(qx[mm][0] * eo[0], qx[mm][1] * eo[1]);
                const uint32_t aq1 = pack2bf(qx[mm][2] * eo[2], qx[mm][3] * eo[3]);
                const float av[4] = {bf_lo(ak0), bf_hi(ak0), bf_lo(ak1), bf_hi(ak1)};
                const float aqv[4] = {bf_lo(aq0), bf_hi(aq0), bf_lo(aq1), bf_hi(aq1)};
                const Frag4 Ak{__builtin_bit_cast(short4v, make_uint2(ak0, ak1)), short4v{0, 0, 0, 0}};
                const Frag4 Aq{__builtin_bit_cast(short4v, make_uint2(aq0, aq1)), short4v{0, 0, 0, 0}};
                // row-side A operands (rows t = 16 m + r16) and column-side A
                // operands (rows s = 16 m + r16, k = t = 16 m + 4 g + e)
                const float bi = s.beta[BS * m + r16];
                const float4 x = *reinterpret_cast<const float4*>(sdL + (BS * m + r16) * LDL + BS * m + 4 * g4);
                const float pr[4] = {bi * x.x, bi * x.y, bi * x.z, bi * x.w};
                // (dA is strictly lower: the diagonal pairs are added apart, below)
                Frag4 Ar = frag4_from_f32<1>(pr), Aqr = ldfrag4<1, ST>(&sm.dA[0][0], LDT, BS * m, BS * m);
                float pc[4], ac[4];
                short4v acr;   // bf16 dA: its raw halves are the fragment
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * m + 4 * g4 + e;
                    pc[e] = s.beta[t] * sdL[t * LDL + BS * m + r16];
                    if constexpr (std::is_same<ST, uint16_t>::value)
                        acr[e] = (short)sm.dA[t][BS * m + r16];
                    else
                        ac[e] = ld1<ST>(&sm.dA[t][BS * m + r16]);
                }
                const Frag4 Ac = frag4_from_f32<1>(pc);
                Frag4 Aqc;
                if constexpr (std::is_same<ST, uint16_t>::value) Aqc = Frag4{acr, short4v{0, 0, 0, 0}};
                else Aqc = frag4_from_f32<1>(ac);
                const Frag4 z4{short4v{0, 0, 0, 0}, short4v{0, 0, 0, 0}};
                f32x4 rk = zero4(), rq = zero4();
                float ck[4] = {0.f, 0.f, 0.f, 0.f}, cg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int p = 0; p < NB; ++p) {
                    float f[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) f[e] = wp[p] * vt[e];
                    const uint32_t b0 = pack2bf(kx[mm][0] * f[0], kx[mm][1] * f[1]);
                    const uint32_t b1 = pack2bf(kx[mm][2] * f[2], kx[mm][3] * f[3]);
                    const float bv[4] = {bf_lo(b0), bf_hi(b0), bf_lo(b1), bf_hi(b1)};
                    const Frag4 Bp{__builtin_bit_cast(short4v, make_uint2(b0, b1)), short4v{0, 0, 0, 0}};
                    const bool rowp = (r16 >> 2) == p, colp = g4 == p;
                    rk = mma4f<1>(rowp ? Ar : z4, Bp, rk);
                    rq = mma4f<1>(rowp ? Aqr : z4, Bp, rq);
                    f32x4 c = mma4f<1>(Ac, colp ? Ak : z4, zero4());
                    c = mma4f<1>(Aqc, colp ? Aq : z4, c);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ck[e] += c[e] * f[e];
                        cg[e] += c[e] * bv[e];
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dka[mm][e] += rk[e] * eo[e] + ck[e];
                    dqa[mm][e] += rq[e] * eo[e];
                    dga[mm][e] += rk[e] * av[e] + rq[e] * aqv[e] - cg[e];
                }
            }
            // Diagonal tiles of own blocks in qmask (4-row spans beyond the guard
            // too), pair by pair with the exact weight e^{a_t - a_s}, from the
            // raw k, q and a of the block's rows (shuffled from the lanes that own
            // them).  Row side (s < t) and column side (s > t) of each own row t;
            // the diagonal s = t is added apart, below.
#pragma unroll
            for (int mm = 0; mm < MB; ++mm) {
                const int m = 2 * rh + mm;
                if (!((qmask >> m) & 1)) continue;
                float ak[4] = {0.f, 0.f, 0.f, 0.f}, aq[4] = {0.f, 0.f, 0.f, 0.f}, ag[4] = {0.f, 0.f, 0.f, 0.f};
                // a rolled loop (rare path, kept compact): the source register is picked by selects
#pragma unroll 1
                for (int sq = 0; sq < BS; ++sq) {
                    const int src = 16 * (sq >> 2) + r16, sr = BS * m + sq, es = sq & 3;
                    const float kv = (es == 0) ? kx[mm][0] : (es == 1) ? kx[mm][1] : (es == 2) ? kx[mm][2] : kx[mm][3];
                    const float qv = (es == 0) ? qx[mm][0] : (es == 1) ? qx[mm][1] : (es == 2) ? qx[mm][2] : qx[mm][3];
                    const float av = (es == 0) ? at[mm][0] : (es == 1) ? at[mm][1] : (es == 2) ? at[mm][2] : at[mm][3];
                    const float Ks = __shfl(kv, src, 64);
                    const float Qs = __shfl(qv, src, 64);
                    const float As = __shfl(av, src, 64);
                    const float bs = s.beta[sr];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int tr = 4 * g4 + e, t = BS * m + tr;
                        if (sq < tr) {
                            const float ks = Ks * kexp<PREC>(at[mm][e] - As);
                            const float pp = s.beta[t] * sdL[t * LDL + sr], pa = ld1<ST>(&sm.dA[t][sr]);
                            ak[e] += pp * ks;
                            aq[e] += pa * ks;
                            ag[e] += (pp * kx[mm][e] + pa * qx[mm][e]) * ks;
                        } else if (sq > tr) {
                            const float pp = bs * sdL[sr * LDL + t], pa = ld1<ST>(&sm.dA[sr][t]);
                            const float c = (pp * Ks + pa * Qs) * kexp<PREC>(As - at[mm][e]);
                            ak[e] += c;
                            ag[e] -= c * kx[mm][e];
                        }
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dka[mm][e] += ak[e];
                    dqa[mm][e] += aq[e];
                    dga[mm][e] += ag[e];
                }
            }
        } else {
            // every pair pairwise (g > 0 or NaN in the chunk): raw k in kr, raw q in
            // ql, a in g.  Row side (s < t) and column side (s > t) as two loops.
#pragma unroll
            for (int mm = 0; mm < MB; ++mm)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * (2 * rh + mm) + 4 * g4 + e;
                    const float gt = chunk_gamma(s, t, d), bt = s.beta[t];
                    float ak = 0.f, aq = 0.f, ag = 0.f;
#pragma unroll 1
                    for (int sx = 0; sx < t; ++sx) {
                        const float ks = ld1<ST>(&s.kr[sx][d]) * kexp<PREC>(gt - chunk_gamma(s, sx, d));
                        const float pp = bt * sdL[t * LDL + sx], pa = ld1<ST>(&sm.dA[t][sx]);
                        ak += pp * ks;
                        aq += pa * ks;
                        ag += (pp * kx[mm][e] + pa * qx[mm][e]) * ks;
                    }
#pragma unroll 1
                    for (int sx = t + 1; sx < C; ++sx) {
                        const float ex = kexp<PREC>(chunk_gamma(s, sx, d) - gt);
                        const float pp = s.beta[sx] * sdL[sx * LDL + t], pa = ld1<ST>(&sm.dA[sx][t]);
                        const float c = (pp * ld1<ST>(&s.kr[sx][d]) + pa * ld1<ST>(&s.ql[sx][d])) * ex;
                        ak += c;
                        ag -= c * kx[mm][e];
                    }
                    dka[mm][e] += ak;
                    dqa[mm][e] += aq;
                    dga[mm][e] += ag;
                }
        }
        // The diagonal pairs (t, t) of A_qk (weight e^0 = 1): dq_t += dA_tt k_t and
        // dk_t += dA_tt q_t.  Their row and column terms of dgamma_t are equal and
        // opposite, so they are left out of it altogether: summed into the row and
        // column sides they would dominate both (the off-diagonal pairs carry
        // decayed weights), and the fp32 rounding of those sums, relative to the
        // diagonal term, would survive the cancellation into dg.
#pragma unroll
        for (int mm = 0; mm < MB; ++mm)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * (2 * rh + mm) + 4 * g4 + e;
                const float a = ld1<ST>(&sm.dA[t][C]);
                dqa[mm][e] += a * kx[mm][e];
                dka[mm][e] += a * qx[mm][e];
            }
    }

    // ---------------- phase 5: dG, reverse cumsum over the two row halves ----------------
    float lsum[MB][4];
    if (own) {
        if (rh == 1 && g4 == 3)      // row C-1
            dga[MB - 1][3] += dgcol + xg[d];
        float tot[MB];
#pragma unroll
        for (int mm = 0; mm < MB; ++mm) {
            float run = 0.f;
#pragma unroll
            for (int e = 3; e >= 0; --e) { run += dga[mm][e]; lsum[mm][e] = run; }
            tot[mm] = run;
        }
        float after_m = 0.f;
#pragma unroll
        for (int mm = MB - 1; mm >= 0; --mm) {
            const float t0v = __shfl(tot[mm], r16, 64);
            const float t1v = __shfl(tot[mm], r16 + 16, 64);
            const float t2v = __shfl(tot[mm], r16 + 32, 64);
            const float t3v = __shfl(tot[mm], r16 + 48, 64);
            const float later = (g4 < 1 ? t1v : 0.f) + (g4 < 2 ? t2v : 0.f) + (g4 < 3 ? t3v : 0.f);
#pragma unroll
            for (int e = 0; e < 4; ++e) lsum[mm][e] += later + after_m;
            after_m += t0v + t1v + t2v + t3v;
        }
        if (rh == 1 && g4 == 0) xt[d] = after_m;     // total over rows 32..63
    }
    __syncthreads();   // xt; region A (dR) and B (dL) dead
    // GH (one decay per (b, t, h)): dg of a row is the sum of its channels'
    // values, in fp32: over the 16 channels of the wave's tile by lane shuffles,
    // then over the tiles through gpart[ct][t] (in the dg staging tile's bytes)
    constexpr bool GH = std::is_same<TG, GHead>::value;
    float* gpart = reinterpret_cast<float*>(&sm.ra.out[3][0][0]);
    static_assert(!GH || 4 * C * 4 <= (int)sizeof(sm.ra.out[3]), "dg partials fit the dg staging tile");
    if (own) {
        const float add = rh == 0 ? xt[d] : 0.f;
#pragma unroll
        for (int mm = 0; mm < MB; ++mm)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * (2 * rh + mm) + 4 * g4 + e;
                st1<ST>(&sm.ra.out[0][t][d], dqa[mm][e]);
                st1<ST>(&sm.ra.out[1][t][d], dka[mm][e]);
                st1<ST>(&sm.ra.out[2][t][d], dvo[mm][e]);
                if constexpr (GH) {
                    const float rsum = sum16(lsum[mm][e] + add);
                    if (r16 == 0) gpart[ct * C + t] = rsum;
                } else if constexpr (std::is_same<TG, ST>::value) {
                    st1<ST>(&sm.ra.out[3][t][d], lsum[mm][e] + add);
                } else if (t < valid) {
                    // fp32 g with bf16 operands: dg in fp32 straight from the
                    // registers (16 lanes write 64 contiguous bytes), not
                    // through the bf16 staging tile
                    st1<TG>(static_cast<TG*>(a.dg) + base + (size_t)t * rs + d, lsum[mm][e] + add);
                }
            }
    }
    __syncthreads();
    dma_wait<0>();   // the prefetch has landed (issued thousands of cycles ago)
    tile_out<ST, C, D, NTH>(&sm.ra.out[0][0][0], LDK, static_cast<ST*>(a.dq) + base, rs, valid);
    tile_out<ST, C, D, NTH>(&sm.ra.out[1][0][0], LDK, static_cast<ST*>(a.dk) + base, rs, valid);
    tile_out<ST, C, D, NTH>(&sm.ra.out[2][0][0], LDK, static_cast<ST*>(a.dv) + base, rs, valid);
    if constexpr (GH) {
        if (tid < valid) {
            float x = 0.f;
#pragma unroll
            for (int c2 = 0; c2 < NT; ++c2) x += gpart[c2 * C + tid];
            static_cast<float*>(a.dg)[bbase + (size_t)tid * a.H] = x;
        }
    } else if constexpr (std::is_same<TG, ST>::value) {
        tile_out<ST, C, D, NTH>(&sm.ra.out[3][0][0], LDK, static_cast<ST*>(a.dg) + base, rs, valid);
    }
    if (tid < valid) st1<ST>(static_cast<ST*>(a.dbeta) + bbase + (size_t)tid * a.H, sm.dbeta[tid]);
}

// The bf16 local-adjoint kernel: phase 0 (loads), the in-block cumsum and the
// factor tables, then local3_tail above.
template <int D, typename ST, typename TG, int PREC>
__global__ __launch_bounds__(512) void kda_bwd_local3_kernel(const LocalArgs a) {
    using L = LocalSmem<D, ST>;
    constexpr int NTH = 512, LDK = L::LDK;
    __shared__ L sm;
    __shared__ float xg[D];     // dgamma(C-1) partial of the rh = 0 waves
    __shared__ float xt[D];     // dgamma column totals of the rh = 1 waves
    __shared__ __align__(16) char pfbuf[256];   // landing bytes of the L2 prefetch
    auto& s = sm.s;

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15,
              g4 = l >> 4;
    __builtin_assume(w >= 0 && w < 8);
    const int ct = w & 3, rh = w >> 2;
    const int ch = blockIdx.x, bh = ch / a.nc, n = ch - bh * a.nc;
    const int b = bh / a.H, h = bh - b * a.H;
    const int t0 = n * C, valid = min(C, a.T - t0);
    const size_t rs = (size_t)a.H * D;
    const size_t base = ((size_t)b * a.T + t0) * rs + (size_t)h * D;
    const size_t bbase = ((size_t)b * a.T + t0) * a.H + h;
    const size_t cCD = (size_t)ch * C * D, cDD = (size_t)ch * D * D;
    // one LDS word for the workgroup's decay flags: a pad column of akk, never data
    int* flagw = reinterpret_cast<int*>(&sm.akk[0][C]);

    // ---------------- phase 0: loads ----------------
    // All loads are issued here, in the order they are needed (q, k, g, beta of
    // all waves first); only q, k, g and beta are waited for before the cumsum.  W, U, h and the phase-1
    // operands stay in registers (4 per thread per tile) until the cumsum and the
    // anchored transform are done, so their latency hides behind those phases.
    // g is loaded as lane (row 16 b + r16 of block b, 8 channels): the 16 rows of
    // a block and 8 channels sit in the 16 lanes of one DPP row, so that the
    // in-block cumsum a is a four-step lane scan before g reaches LDS.
    int flag = 0;
    Local3Tiles<D, ST> tl;
    auto &tW = tl.W, &tU = tl.U, &tdo = tl.dO, &tv = tl.v, &tdVp = tl.dVp;
    auto &th = tl.h, &tdh = tl.dh;
    float braw;
    {
        Tile<ST, C, D, NTH> tq, tk;
        // GH: one decay per (b, t, h), read once per row
        constexpr bool GH = std::is_same<TG, GHead>::value;
        using TGE = typename std::conditional<GH, float, TG>::type;
        constexpr int NCG = D / 8, WPB = NCG / 4, GV = GH ? 1 : 8 * (int)sizeof(TGE) / 16,
                      GE = 16 / (int)sizeof(TGE);
        static_assert(NCG % 4 == 0 && NB * WPB <= 8, "one lane per row and 8 channels of g");
        const bool gl = w < NB * WPB;
        const int grow = BS * (w / WPB) + r16, gc = 8 * (4 * (w % WPB) + g4);
        uint4 graw[GV];
        float gh = 0.f;
        tq.load(static_cast<const ST*>(a.q) + base, rs, valid);
        tk.load(static_cast<const ST*>(a.k) + base, rs, valid);
        if (gl) {
            if constexpr (GH) {
                gh = static_cast<const float*>(a.g)[bbase + (size_t)min(grow, valid - 1) * a.H];
            } else {
                const TGE* gp = static_cast<const TGE*>(a.g) + base + (size_t)min(grow, valid - 1) * rs + gc;
#pragma unroll
                for (int vq = 0; vq < GV; ++vq) graw[vq] = *reinterpret_cast<const uint4*>(gp + GE * vq);
            }
        }
        braw = ld1<ST>(static_cast<const ST*>(a.beta) + bbase + (size_t)min(tid, valid - 1) * a.H);
        // Every wave's q, k, g, beta requests enter the CU's memory pipeline before
        // any wave's later tiles, so no wave waits behind another's 80 KB.
        __builtin_amdgcn_s_barrier();
        tW.load(static_cast<const ST*>(a.W) + cCD, D);
        tU.load(static_cast<const ST*>(a.U) + cCD, D);
        th.load(static_cast<const ST*>(a.h) + cDD, D);
        tdo.load(static_cast<const ST*>(a.dout) + base, rs, valid);
        tv.load(static_cast<const ST*>(a.v) + base, rs, valid);
        tdVp.load(static_cast<const ST*>(a.dVp) + cCD, D);
        tdh.load(static_cast<const ST*>(a.dh) + cDD, D);
        tq.store(&s.ql[0][0], LDK);
        tk.store(&s.kr[0][0], LDK);
        if (gl) {
            // rows past T read as zero; a = in-block inclusive cumsum of g
            float x[8];
            if constexpr (GH) {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = (grow < valid) ? gh : 0.f;
            } else {
#pragma unroll
                for (int vq = 0; vq < GV; ++vq) {
                    const Vec16<TGE> xv{graw[vq]};
#pragma unroll
                    for (int e = 0; e < GE; ++e) x[GE * vq + e] = (grow < valid) ? xv.get(e) : 0.f;
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (!(x[e] <= 0.f)) flag = 1;
                x[e] = row16_scan(x[e]);
            }
            *reinterpret_cast<float4*>(&s.g[grow][gc]) = make_float4(x[0], x[1], x[2], x[3]);
            *reinterpret_cast<float4*>(&s.g[grow][gc + 4]) = make_float4(x[4], x[5], x[6], x[7]);
        }
        if (tid < C) sm.dbeta[tid] = 0.f;
        if (tid == 0) *flagw = 0;
    }
    __syncthreads();
    const int dfl = chunk_factors2<D, ST, PREC, NTH>(s, flag, flagw);
    // The rest is instantiated twice.  Chunks whose 16-row blocks all stay within
    // the span guard (every chunk at ordinary decays) run a copy with the
    // sub-anchored and pairwise code compiled out, so that code shapes neither
    // that copy's register allocation nor its schedule.
    Local3Chunk c{tid, w, l, r16, g4, ct, rh, valid, rs, base, bbase, {nullptr}};
    // L2 prefetch of the chunk this XCD starts next (chunks a CU count apart go to
    // one XCD and start about when this one ends): one 4-byte DMA per 128-byte
    // line of the rows of q, k and g, the inputs a chunk waits for before its
    // cumsum, so that those loads hit in L2 (without it the kernel takes 4% longer).
    // The other inputs' latency hides behind the cumsum and factor phases:
    // prefetching them as well (80 KB per chunk in all) gave no gain and more
    // lines evicted before use.  The addresses are formed here, from the argument
    // block; the tail issues the DMA once the chunk's own loads are in.
    if (a.pf_ahead > 0 && ch + a.pf_ahead < (int)gridDim.x) {
        const int pc = ch + a.pf_ahead, pbh = pc / a.nc, pn = pc - pbh * a.nc;
        const int pb = pbh / a.H, ph = pbh - pb * a.H, pt0 = pn * C, pvalid = min(C, a.T - pt0);
        const size_t pbase = ((size_t)pb * a.T + pt0) * rs + (size_t)ph * D;
        // (a decay per (b, t, h) is 4 bytes a row: not worth a line each)
        constexpr int NL = (std::is_same<TG, GHead>::value ? 2 : 3) * C;
        static_assert((NL + NTH - 1) / NTH <= Local3Chunk::NPF, "prefetch lines per thread");
#pragma unroll
        for (int i = 0; i < (NL + NTH - 1) / NTH; ++i) {
            const int k = NTH * i + tid;
            const char* p = nullptr;
            if (k < NL) {
                const int ts = k / C, r = k - ts * C;
                const char* tp = static_cast<const char*>(ts == 0 ? a.q : ts == 1 ? a.k : a.g);
                const size_t es = (ts == 2) ? sizeof(typename std::conditional<std::is_same<TG, GHead>::value, float, TG>::type)
                                            : sizeof(ST);
                if (r < pvalid) p = tp + (pbase + (size_t)r * rs) * es;
            }
            c.pf[i] = p;
        }
    }
    if (__builtin_expect((dfl & 31) != 0, 0))
        local3_tail<D, ST, TG, PREC, true>(a, sm, xg, xt, pfbuf, c, tl, braw, dfl);
    else
        local3_tail<D, ST, TG, PREC, false>(a, sm, xg, xt, pfbuf, c, tl, braw, dfl);
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
template <int D, typename TI, typename TG>
static hipError_t launch_local_t(const LocalArgs& a, int nchunks, hipStream_t st) {
    if constexpr (std::is_same<TI, float>::value)
        hipLaunchKernelGGL((kda_bwd_local_kernel<D, TI, TG, 3>), dim3(nchunks), dim3(256), 0, st, a);
    else {
        // prefetch distance: one chunk per CU (one local-adjoint workgroup fills a CU)
        int dev = 0;
        LocalArgs b = a;
        b.pf_ahead = (hipGetDevice(&dev) == hipSuccess) ? device_cu_count(dev) : 0;
        hipLaunchKernelGGL((kda_bwd_local3_kernel<D, TI, TG, 1>), dim3(nchunks), dim3(512), 0, st, b);
    }
    return hipGetLastError();
}

// g_kind: 0 fp32 g, 1 bf16 g, 2 one fp32 decay per (b, t, h) (bf16 inputs at
// D <= 64 only)
hipError_t launch_local(const LocalArgs& a, int D, int in_bf16, int g_kind, int nchunks, hipStream_t st) {
    if (g_kind == 2) {
        if (!in_bf16) return hipErrorInvalidValue;
        if (D == 32) return launch_local_t<32, uint16_t, GHead>(a, nchunks, st);
        if (D == 64) return launch_local_t<64, uint16_t, GHead>(a, nchunks, st);
        return hipErrorInvalidValue;
    }
    const int g_bf16 = g_kind == 1;
#define KDA_LOCAL_CASE(DD)                                                                         \
    if (D == DD) {                                                                                 \
        if (in_bf16) return g_bf16 ? launch_local_t<DD, uint16_t, uint16_t>(a, nchunks, st)        \
                                   : launch_local_t<DD, uint16_t, float>(a, nchunks, st);          \
        return g_bf16 ? launch_local_t<DD, float, uint16_t>(a, nchunks, st)                        \
                      : launch_local_t<DD, float, float>(a, nchunks, st);                          \
    }
    KDA_LOCAL_CASE(32)
    KDA_LOCAL_CASE(64)
#undef KDA_LOCAL_CASE
    if (D == 128) return launch_local_wide(a, D, in_bf16, g_bf16, nchunks, st);
    return hipErrorInvalidValue;
}

}  // namespace kda
