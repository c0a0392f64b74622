// kda_fwd.hip -- forward kernels of the KDA chunkwise WY recurrence (gfx950).
//
//   kda_prep_kernel   one workgroup per (batch, head, chunk), fully parallel.
//                     In-chunk cumsum gamma, decay-masked Akk = tril(K K^T . decay, -1)
//                     and Aqk = tril(Q K^T . decay) on bf16 MFMA (anchored 16-row
//                     sub-blocks), L = diag(beta) Akk, inverted 16x16 diagonal
//                     blocks of I + L held in LDS, block forward substitution
//                     [W | U] = (I + L)^-1 [beta e^gamma K | beta V], plus
//                     Qp = e^gamma Q, Kb = e^(G - gamma) K and e^G.
//                     Replaces nope_gdn_mlx.py:549-597 (preamble, M / M_oq
//                     kernels 1301-1469, IA build) and lifts the triangular solve
//                     (1098-1196) out of the sequential chunk loop.
//   kda_recur_kernel  one wave per (batch, head, 16-column dv tile), sequential
//                     over chunks, state tile resident in accumulator VGPRs:
//                         V' = U - W S;  O = Qp S + Aqk V';  S <- e^G S + Kb^T V'
//                     (S in [dk, dv] orientation).  Replaces the per-chunk
//                     solve/finalize launches (nope_gdn_mlx.py:1519-1942,
//                     2408-2451).  MODE 1 stores chunk-start states and V' for
//                     the backward instead of the output.
#include "kda_internal.h"

namespace kda {

// ----------------------------------------------------------------------------
// prep
// ----------------------------------------------------------------------------
template <int D, typename TI, typename TG, int PREC>
__global__ __launch_bounds__(256) void kda_prep_kernel(const PrepArgs a) {
    __shared__ ChunkLds<D> s;
    __shared__ float sl[C][C + 4];            // L = diag(beta) Akk (strict lower)
    __shared__ float tii[NB][BS][BS + 4];     // (I + L_ii)^-1

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
    const size_t cCD = (size_t)ch * C * D, cCC = (size_t)ch * C * C;

    int flag = chunk_load<D, TI, TG>(s, q, k, g, beta, base, rs, bbase, a.H, valid);
    chunk_cumsum<D>(s);
    const int unsafe = chunk_factors<D, PREC>(s, flag);

    if (unsafe) {
        // pairwise path (reference M kernel order of operations, any decay)
        for (int p = tid; p < C * C; p += 256) {
            const int t = p / C, sx = p - t * C;
            float ak = 0.f, aq = 0.f;
            if (sx <= t) {
                for (int d = 0; d < D; ++d) {
                    const float e = kexp<PREC>(s.g[t][d] - s.g[sx][d]);
                    const float ks = s.kr[sx][d] * e;
                    ak += s.kr[t][d] * ks;
                    aq += s.ql[t][d] * ks;
                }
            }
            const float akk = (sx < t) ? ak : 0.f;
            sl[t][sx] = s.beta[t] * akk;
            if (a.Akk) a.Akk[cCC + (size_t)t * C + sx] = akk;
            if (a.Aqk) a.Aqk[cCC + (size_t)t * C + sx] = aq;
            if (a.AqkT) a.AqkT[cCC + (size_t)sx * C + t] = aq;
        }
        __syncthreads();
    }

    // elementwise: Qp, Kb, e^G to the workspace; anchored operands in LDS
    for (int idx = tid; idx < C * D; idx += 256) {
        const int t = idx / D, d = idx - t * D;
        const float gt = s.g[t][d], G = s.g[C - 1][d];
        const float qv = s.ql[t][d], kv = s.kr[t][d];
        const float qp = qv * kexp<PREC>(gt);
        const float kb = kv * kexp<PREC>(G - gt);
        if (a.Qp) a.Qp[cCD + (size_t)t * D + d] = qp;
        if (a.QpT) a.QpT[cCD + (size_t)d * C + t] = qp;
        if (a.Kb) a.Kb[cCD + (size_t)t * D + d] = kb;
        if (a.KbT) a.KbT[cCD + (size_t)d * C + t] = kb;
        if (t == 0 && a.eG) a.eG[(size_t)ch * D + d] = kexp<PREC>(G);
    }
    __syncthreads();
    chunk_transform<D, PREC>(s, !unsafe);
    __syncthreads();

    if (!unsafe) {
        // 10 lower sub-block tiles of Akk and Aqk; B operand shared by both
        for (int tix = w; tix < 10; tix += 4) {
            int i, j;
            tile_ij(tix, i, j);
            f32x4 P = zero4(), Q = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                Fr8 Ak = frag8(&s.kl[0][0], D + 4, BS * i, 32 * ks);
                Fr8 Aq = frag8(&s.ql[0][0], D + 4, BS * i, 32 * ks);
                Fr8 Bk = frag8(&s.kr[0][0], D + 4, BS * j, 32 * ks);
                if (j < i) {
                    const float* f = &s.f[pair_idx(i, j)][32 * ks];
#pragma unroll
                    for (int e = 0; e < 8; ++e) Bk.v[e] *= f[kslot(g4, e)];
                }
                P = mma8<PREC>(Ak, Bk, P);
                Q = mma8<PREC>(Aq, Bk, Q);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
                const float akk = (sx < t) ? P[e] : 0.f;
                const float aq = (sx <= t) ? Q[e] : 0.f;
                sl[t][sx] = s.beta[t] * akk;
                if (a.Akk) a.Akk[cCC + (size_t)t * C + sx] = akk;
                if (a.Aqk) a.Aqk[cCC + (size_t)t * C + sx] = aq;
                if (a.AqkT) a.AqkT[cCC + (size_t)sx * C + t] = aq;
            }
        }
        // strictly upper sub-block tiles are zero in the workspace copies
        for (int idx = tid; idx < 6 * BS * BS; idx += 256) {
            const int tile = idx / (BS * BS), e = idx - tile * BS * BS;
            const int i = (tile < 3) ? 0 : (tile < 5) ? 1 : 2;
            const int j = (tile < 3) ? tile + 1 : (tile < 5) ? tile - 1 : 3;
            const int t = BS * i + e / BS, sx = BS * j + (e % BS);
            if (a.Akk) a.Akk[cCC + (size_t)t * C + sx] = 0.f;
            if (a.Aqk) a.Aqk[cCC + (size_t)t * C + sx] = 0.f;
            if (a.AqkT) a.AqkT[cCC + (size_t)sx * C + t] = 0.f;
        }
    }
    __syncthreads();

    diag_inverse<C + 4>(&sl[0][0], tii, NB);
    __syncthreads();
    if (a.Tii) {
        for (int idx = tid; idx < NB * BS * BS; idx += 256) {
            const int i = idx / (BS * BS), e = idx - i * BS * BS;
            a.Tii[(size_t)ch * NB * BS * BS + idx] = tii[i][e / BS][e % BS];
        }
    }

    // block forward substitution, one 16-column tile of [Kt | beta V] at a time
    constexpr int NCT = 2 * D / BS;
    for (int ct = w; ct < NCT; ct += 4) {
        const bool isK = ct < D / BS;
        const int d = (isK ? ct : ct - D / BS) * BS + r16;
        f32x4 X[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            f32x4 Y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = BS * i + 4 * g4 + e;
                float rv;
                if (isK) rv = s.beta[t] * s.er[i][d] * s.kl[t][d];
                else rv = (t < valid) ? s.beta[t] * ld1<TI>(v + base + (size_t)t * rs + d) : 0.f;
                Y[e] = rv;
            }
#pragma unroll
            for (int j = 0; j < i; ++j) {
                Fr4 A = neg(frag4(&sl[0][0], C + 4, BS * i, BS * j));
                Y = mma4<3>(A, acc2frag4(X[j]), Y);
            }
            X[i] = mma4<3>(frag4(&tii[i][0][0], BS + 4, 0, 0), acc2frag4(Y), zero4());
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int tb = BS * i + 4 * g4;
            if (isK) {
#pragma unroll
                for (int e = 0; e < 4; ++e) a.W[cCD + (size_t)(tb + e) * D + d] = X[i][e];
                if (a.WT)
                    *reinterpret_cast<float4*>(&a.WT[cCD + (size_t)d * C + tb]) =
                        make_float4(X[i][0], X[i][1], X[i][2], X[i][3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) a.U[cCD + (size_t)(tb + e) * D + d] = X[i][e];
            }
        }
    }
}

// ----------------------------------------------------------------------------
// recurrence
// ----------------------------------------------------------------------------
template <int D, typename TI, int PREC, int MODE>
__global__ __launch_bounds__(64) void kda_recur_kernel(const RecurArgs a) {
    constexpr int NT = D / BS;
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = bid / NT, ct = bid - bh * NT;
    const int l = threadIdx.x, r16 = l & 15, g4 = l >> 4;
    const int b = bh / a.H, h = bh - b * a.H;
    const int col = ct * BS + r16;

    f32x4 S[NT];
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) {
        if (a.s0) {
            const float4 x = *reinterpret_cast<const float4*>(a.s0 + ((size_t)bh * D + col) * D + BS * mt + 4 * g4);
            S[mt] = f32x4{x.x, x.y, x.z, x.w};
        } else {
            S[mt] = zero4();
        }
    }

    for (int n = 0; n < a.nc; ++n) {
        const size_t ch = (size_t)bh * a.nc + n;
        const float* W = a.W + ch * C * D;
        const float* U = a.U + ch * C * D;
        const float* KbT = a.KbT + ch * C * D;
        const float* eG = a.eG + ch * D;

        f32x4 Vp[NB];
#pragma unroll
        for (int m = 0; m < NB; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) Vp[m][e] = U[(size_t)(BS * m + 4 * g4 + e) * D + col];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                Vp[m] = mma8<PREC>(neg(frag8(W, D, BS * m, 32 * ks)), acc2frag(S[2 * ks], S[2 * ks + 1]), Vp[m]);
        }

        if constexpr (MODE == 0) {
            const float* Qp = a.Qp + ch * C * D;
            const float* Aqk = a.Aqk + ch * C * C;
            const int t0 = n * C, valid = min(C, a.T - t0);
            TI* o = static_cast<TI*>(a.o);
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                f32x4 O = zero4();
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks)
                    O = mma8<PREC>(frag8(Qp, D, BS * m, 32 * ks), acc2frag(S[2 * ks], S[2 * ks + 1]), O);
#pragma unroll
                for (int ks = 0; ks <= m / 2; ++ks)
                    O = mma8<PREC>(frag8(Aqk, C, BS * m, 32 * ks), acc2frag(Vp[2 * ks], Vp[2 * ks + 1]), O);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * m + 4 * g4 + e;
                    if (t < valid) st1<TI>(o + (((size_t)b * a.T + t0 + t) * a.H + h) * D + col, O[e]);
                }
            }
        } else {
            float* hh = a.h + ch * D * D;
            float* vp = a.Vp + ch * C * D;
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) hh[(size_t)(BS * mt + 4 * g4 + e) * D + col] = S[mt][e];
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) vp[(size_t)(BS * m + 4 * g4 + e) * D + col] = Vp[m][e];
        }

#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            const float4 eg = *reinterpret_cast<const float4*>(eG + BS * mt + 4 * g4);
            S[mt][0] *= eg.x; S[mt][1] *= eg.y; S[mt][2] *= eg.z; S[mt][3] *= eg.w;
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks)
                S[mt] = mma8<PREC>(frag8(KbT, C, BS * mt, 32 * ks), acc2frag(Vp[2 * ks], Vp[2 * ks + 1]), S[mt]);
        }
    }

    if (MODE == 0 && a.s_final) {
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
            *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + col) * D + BS * mt + 4 * g4) =
                make_float4(S[mt][0], S[mt][1], S[mt][2], S[mt][3]);
    }
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
template <int D, typename TI, typename TG>
static hipError_t launch_prep_t(const PrepArgs& a, int nchunks, hipStream_t st) {
    constexpr int PREC = std::is_same<TI, float>::value ? 3 : 1;
    hipLaunchKernelGGL((kda_prep_kernel<D, TI, TG, PREC>), dim3(nchunks), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int D, typename TI>
static hipError_t launch_recur_t(const RecurArgs& a, int mode, hipStream_t st) {
    constexpr int PREC = std::is_same<TI, float>::value ? 3 : 1;
    const dim3 grid(a.BH * (D / BS));
    if (mode == 0) hipLaunchKernelGGL((kda_recur_kernel<D, TI, PREC, 0>), grid, dim3(64), 0, st, a);
    else hipLaunchKernelGGL((kda_recur_kernel<D, TI, PREC, 1>), grid, dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_prep(const PrepArgs& a, int D, int in_bf16, int g_bf16, int nchunks, hipStream_t st) {
#define KDA_PREP_CASE(DD)                                                                          \
    if (D == DD) {                                                                                 \
        if (in_bf16) return g_bf16 ? launch_prep_t<DD, uint16_t, uint16_t>(a, nchunks, st)         \
                                   : launch_prep_t<DD, uint16_t, float>(a, nchunks, st);           \
        return g_bf16 ? launch_prep_t<DD, float, uint16_t>(a, nchunks, st)                         \
                      : launch_prep_t<DD, float, float>(a, nchunks, st);                           \
    }
    KDA_PREP_CASE(32)
    KDA_PREP_CASE(64)
    KDA_PREP_CASE(128)
#undef KDA_PREP_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_recur(const RecurArgs& a, int D, int in_bf16, int mode, hipStream_t st) {
    if (D == 32) return in_bf16 ? launch_recur_t<32, uint16_t>(a, mode, st) : launch_recur_t<32, float>(a, mode, st);
    if (D == 64) return in_bf16 ? launch_recur_t<64, uint16_t>(a, mode, st) : launch_recur_t<64, float>(a, mode, st);
    if (D == 128) return in_bf16 ? launch_recur_t<128, uint16_t>(a, mode, st) : launch_recur_t<128, float>(a, mode, st);
    return hipErrorInvalidValue;
}

}  // namespace kda
