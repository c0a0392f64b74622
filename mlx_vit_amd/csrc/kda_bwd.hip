// kda_bwd.hip -- backward kernels of the KDA chunkwise WY recurrence (gfx950).
//
// The backward stores no per-step state.  The forward's chunk-boundary states
// are recomputed (prep + kda_recur_kernel MODE 1), then:
//
//   kda_dh_kernel     one wave per (batch, head, dv tile), reverse over chunks:
//                         dV' = Aqk^T dO + Kb dS;  dS <- e^G dS + Qp^T dO - W^T dV'
//                     storing dS at each chunk end and dV'; the final dS is dS0.
//                     This is the reverse state carry of nope_gdn_mlx.py:2705-2706.
//   kda_bwd_local_kernel
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
    __shared__ float sdb[C];                 // dbeta

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
    if (tid < C) sdb[tid] = 0.f;
    int flag = chunk_load<D, TI, TG>(s, q, k, g, beta, base, rs, bbase, a.H, valid);
    chunk_cumsum<D>(s);
    const int unsafe = chunk_factors<D, PREC>(s, flag);

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
                if (r16 == 0) atomicAdd(&sdb[t], db);
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
            if (r16 == 0) atomicAdd(&sdb[t], db);
            sp[t][sx] = s.beta[t] * dL;
        }
    }
    __syncthreads();

    // PHASE 4
    // ---------------- phase 4: decay-masked K K^T / Q K^T adjoints ----------------
    if (own) {
        if (!unsafe) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                f32x4 dKl = zero4(), dQl = zero4();
#pragma unroll
                for (int j = 0; j <= i; ++j) {
                    const float fs = (j < i) ? s.f[pair_idx(i, j)][d] : 1.f;
                    Fr4 B;
#pragma unroll
                    for (int e = 0; e < 4; ++e) B.v[e] = s.kr[BS * j + 4 * g4 + e][d] * fs;
                    dKl = mma4<PREC>(frag4(&sp[0][0], C + 4, BS * i, BS * j), B, dKl);
                    dQl = mma4<PREC>(frag4(&sda[0][0], C + 4, BS * i, BS * j), B, dQl);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dka[i][e] += dKl[e] * el[i][e];
                    dqa[i][e] += dQl[e] * el[i][e];
                    dga[i][e] += (dKl[e] * kx[i][e] + dQl[e] * qx[i][e]) * el[i][e];
                }
                Fr4 Bk, Bq;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    Bk.v[e] = s.kl[BS * i + 4 * g4 + e][d];
                    Bq.v[e] = s.ql[BS * i + 4 * g4 + e][d];
                }
#pragma unroll
                for (int j = 0; j <= i; ++j) {
                    f32x4 dKr = mma4<PREC>(frag4T(&sp[0][0], C + 4, BS * j, BS * i), Bk, zero4());
                    dKr = mma4<PREC>(frag4T(&sda[0][0], C + 4, BS * j, BS * i), Bq, dKr);
                    const float fs = (j < i) ? s.f[pair_idx(i, j)][d] : 1.f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float fac = fs * er[j][e];
                        dka[j][e] += dKr[e] * fac;
                        dga[j][e] -= dKr[e] * kx[j][e] * fac;
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
                    for (int sx = 0; sx < C; ++sx) {
                        const float gs = s.g[sx][d];
                        if (sx <= t) {      // row t: dP[t][sx] (strict), dA[t][sx]
                            const float ex = kexp<PREC>(gt - gs);
                            const float ks = s.kr[sx][d] * ex;
                            const float pp = sp[t][sx], pa = sda[t][sx];
                            ak += pp * ks;
                            aq += pa * ks;
                            ag += (pp * kx[m][e] + pa * qx[m][e]) * ks;
                        }
                        if (sx >= t) {      // column t: dP[sx][t] (strict), dA[sx][t]
                            const float ex = kexp<PREC>(gs - gt);
                            const float pp = sp[sx][t], pa = sda[sx][t];
                            const float c = (pp * s.kr[sx][d] + pa * s.ql[sx][d]) * ex;
                            ak += c;
                            ag -= c * kx[m][e];
                        }
                    }
                    dka[m][e] += ak;
                    dqa[m][e] += aq;
                    dga[m][e] += ag;
                }
            }
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
    if (tid < valid) st1<TI>(static_cast<TI*>(a.dbeta) + bbase + (size_t)tid * a.H, sdb[tid]);
    // PHASE 6
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
template <int D, typename TI, typename TG>
static hipError_t launch_local_t(const LocalArgs& a, int nchunks, hipStream_t st) {
    constexpr int PREC = std::is_same<TI, float>::value ? 3 : 1;
    hipLaunchKernelGGL((kda_bwd_local_kernel<D, TI, TG, PREC>), dim3(nchunks), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_local(const LocalArgs& a, int D, int in_bf16, int g_bf16, int nchunks, hipStream_t st) {
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
    return hipErrorInvalidValue;
}

}  // namespace kda
