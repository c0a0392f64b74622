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
// The sequential half of the forward, kda_recur_kernel, is in kda_recur.hip.
#include "kda_internal.h"

namespace kda {

// ----------------------------------------------------------------------------
// prep
//
// Phases (barriers between them):
//   load      all 16-byte loads of q, k, g (and v) issued first, then LDS;
//             a (in-block cumsums of g) by a lane scan on the way
//   factors   factor tables; decay flags: the
//             chunk's g > 0 / NaN, the diagonal blocks beyond the span guard
//   diagonal  those blocks' diagonal tiles from raw q, k: 4-row sub-anchors on
//             MFMA, or pair by pair beyond the 4-row guard too (every pair for
//             a chunk with g > 0)
//   pass A    row-major threads (t, 8 channels): block-end anchored operands
//             kl, ql, kr in place; Qp, Kb (where requested) as 16-byte stores
//   pass B    column threads (d, 8 tokens): KbT, QpT as 16-byte stores
//   products  Akk -> fp32 LDS, Aqk -> LDS staging -> coalesced stores
//   inverse   diagonal 16x16 blocks of I + L in registers (eight waves: waves
//             0-3 form and invert the diagonal tiles beside the products of
//             waves 4-7)
//   solve     block forward substitution, every tile of a wave interleaved;
//             W, U (and WT) staged in LDS, stored coalesced
// ----------------------------------------------------------------------------
template <int D, typename ST>
struct PrepGeom {
    using CSm = ChunkSmem<D, ST>;
    static constexpr int PS = CSm::PS, LDK = CSm::LDK, LDA = C + 4, LDT = C + PS;
    static constexpr int BASE = (int)sizeof(CSm) + C * LDA * 4 + NB * BS * (BS + 4) * 4;
    static constexpr bool STAGE_V = BASE + C * LDK * (int)sizeof(ST) <= 160 * 1024;
    static constexpr bool STG_IN_G = (int)sizeof(float) * C * CSm::LDG >= C * LDT * (int)sizeof(ST);
};

template <int D, typename ST, typename TG, int PREC, int NTH>
__global__ __launch_bounds__(NTH) void kda_prep_kernel(const PrepArgs a) {
    using G = PrepGeom<D, ST>;
    constexpr int NW = NTH / 64;   // waves
    static_assert(NW == 4 || NW == 8 || NW == 16, "four, eight or sixteen waves");
    constexpr int LDK = G::LDK, LDA = G::LDA, LDT = G::LDT, NT = D / BS, NCT = 2 * NT;
    constexpr int TPW = (NCT + NW - 1) / NW;
    constexpr int EPV = 16 / (int)sizeof(ST);
    __shared__ ChunkSmem<D, ST> s;
    __shared__ __align__(16) float sa[C][LDA];            // Akk, fp32, strictly lower, unscaled
    __shared__ __align__(16) float tii[NB][BS][BS + 4];   // (I + L_ii)^-1
    __shared__ __align__(16) ST svbuf[G::STAGE_V ? C : 1][G::STAGE_V ? LDK : 8];
    __shared__ __align__(16) ST stgbuf[G::STG_IN_G ? 1 : C][G::STG_IN_G ? 8 : LDT];

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, g4 = l >> 4;
    __builtin_assume(w >= 0 && w < NW);
    const int ch = blockIdx.x, bh = ch / a.nc, n = ch - bh * a.nc;
    const int b = bh / a.H, h = bh - b * a.H;
    const int t0 = n * C, valid = min(C, a.T - t0);
    // dio: the channels of a q, k, v, g row (< D only at D = 128: the rest read as zero)
    const int dio = (D == 128 && a.dio > 0) ? a.dio : D;
    const size_t rs = (size_t)a.H * dio;
    const size_t base = ((size_t)b * a.T + t0) * rs + (size_t)h * dio;
    const size_t bbase = ((size_t)b * a.T + t0) * a.H + h;
    const ST* q = static_cast<const ST*>(a.q);
    const ST* k = static_cast<const ST*>(a.k);
    const ST* v = static_cast<const ST*>(a.v);
    const TG* g = static_cast<const TG*>(a.g);
    const ST* beta = static_cast<const ST*>(a.beta);
    const size_t cCD = (size_t)ch * C * D, cCC = (size_t)ch * C * C;
    ST* oW = static_cast<ST*>(a.W);
    ST* oU = static_cast<ST*>(a.U);
    ST* oQp = static_cast<ST*>(a.Qp);
    ST* oQpT = static_cast<ST*>(a.QpT);
    ST* oKb = static_cast<ST*>(a.Kb);
    ST* oKbT = static_cast<ST*>(a.KbT);
    ST* oWT = static_cast<ST*>(a.WT);
    ST* oAqk = static_cast<ST*>(a.Aqk);
    ST* oAqkT = static_cast<ST*>(a.AqkT);
    // four consecutive elements of a transposed output row, straight from an MFMA
    // accumulator (lane (g, n) holds rows 4 g .. 4 g + 3 of column n)
    auto st4 = [](ST* p, const float* x) __attribute__((always_inline)) {
        if constexpr (std::is_same<ST, uint16_t>::value)
            *reinterpret_cast<uint2*>(p) = make_uint2(pack2bf(x[0], x[1]), pack2bf(x[2], x[3]));
        else
            *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    };

    // one LDS word for the workgroup's decay flags: a pad column of sa, never data
    int* flagw = reinterpret_cast<int*>(&sa[0][C]);
    if (tid == 0) *flagw = 0;
    // PHASE 0 (load); v stays in registers until the column pass is done
    Tile<ST, C, D, NTH> tv;
    const int flag =
        chunk_load2<D, ST, TG, G::STAGE_V, NTH>(s, tv, q, k, v, g, beta, base, rs, bbase, a.H, valid, dio);
    // PHASE 1
    const int dfl = chunk_factors2<D, ST, PREC, NTH>(s, flag, flagw);
    // The rest of the kernel is instantiated twice.  Chunks whose 16-row blocks
    // all stay within the span guard (every chunk at ordinary decays) run a copy
    // with the sub-anchored and pairwise code compiled out, so that code shapes
    // neither the common copy's register allocation nor its schedule.
    const auto a_Akk = a.Akk;
    const auto a_Tii = a.Tii;
    const auto a_eG = a.eG;
    auto tail = [&](auto strong_c) __attribute__((always_inline)) {
        constexpr bool STRONG = decltype(strong_c)::value;
        const bool unsafe = STRONG && (dfl & 16) != 0;           // g > 0 or NaN: every pair pairwise
        const int pmask = (STRONG && !unsafe) ? (dfl & 15) : 0;  // diagonal blocks beyond the span guard
        if (a_eG && tid < D) {
            const float G = (s.g[BS - 1][tid] + s.g[2 * BS - 1][tid]) + (s.g[3 * BS - 1][tid] + s.g[C - 1][tid]);
            a_eG[(size_t)ch * D + tid] = kexp<PREC>(G);
        }
        // PHASE 2

        // A_qk of the pairwise diagonal-tile entries this thread owns: kept in
        // registers until the tile is staged (the staging buffer may be the g region)
        constexpr int NPW = NB * BS * BS / NTH;
        float paq[NPW], saq[4];
        const int qmask = pmask & (dfl >> 5);           // ... whose 4-row sub-blocks also exceed it
        if (unsafe) {
            // every pair s <= t from raw q (ql), raw k (kr), exact exp(gamma_t - gamma_s)
            for (int p = tid; p < C * C; p += NTH) {
                const int t = p / C, sx = p - t * C;
                float ak = 0.f, aq = 0.f;
                if (sx <= t) {
#pragma unroll 1
                    for (int d = 0; d < D; ++d) {
                        const float ks = ld1<ST>(&s.kr[sx][d]) * kexp<PREC>(chunk_gamma(s, t, d) - chunk_gamma(s, sx, d));
                        ak += ld1<ST>(&s.kr[t][d]) * ks;
                        aq += ld1<ST>(&s.ql[t][d]) * ks;
                    }
                }
                const float akk = (sx < t) ? ak : 0.f;
                sa[t][sx] = akk;
                if (a_Akk) a_Akk[cCC + (size_t)t * C + sx] = akk;
                if (oAqk) st1<ST>(oAqk + cCC + (size_t)t * C + sx, aq);
                if (oAqkT) st1<ST>(oAqkT + cCC + (size_t)sx * C + t, aq);
            }
            __syncthreads();
        } else if (pmask) {
            // Diagonal tiles of the blocks in pmask, from raw q, k (pass A overwrites
            // them).  Wave w forms block w's tile with 4-row sub-anchors on MFMA;
            // blocks whose 4-row sub-blocks also exceed the guard (qmask) are
            // evaluated one entry (t, s) per thread and step, e^{a_t - a_s}.  A_kk
            // goes to sa now (its tile is not formed below), A_qk^T to its output;
            // A_qk stays in registers until its tile is staged.
            if (((pmask & ~qmask) >> w) & 1) {
                f32x4 P, Q;
                subanchor_tile<D, ST, PREC, true>(s, w, P, Q);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * w + 4 * g4 + e, sx = BS * w + r16;
                    sa[t][sx] = (sx < t) ? P[e] : 0.f;
                    saq[e] = (sx <= t) ? Q[e] : 0.f;
                }
                if (oAqkT) st4(oAqkT + cCC + (size_t)(BS * w + r16) * C + BS * w + 4 * g4, saq);
            }
            if (qmask) {
                const int nent = __popc(qmask) * BS * BS;
#pragma unroll
                for (int it = 0; it < NPW; ++it) {
                    const int pp = tid + NTH * it;
                    paq[it] = 0.f;
                    if (pp < nent) {
                        const int kb = pp / (BS * BS), e = pp - kb * BS * BS;
                        int blk = 0;
                        for (int m = qmask, c = 0;; m &= m - 1, ++c)
                            if (c == kb) { blk = __ffs(m) - 1; break; }
                        const int t = BS * blk + e / BS, sx = BS * blk + e % BS;
                        float ak = 0.f, aq = 0.f;
                        if (sx <= t) {
#pragma unroll 2
                            for (int d = 0; d < D; ++d) {
                                const float ks = ld1<ST>(&s.kr[sx][d]) * kexp<PREC>(s.g[t][d] - s.g[sx][d]);
                                ak += ld1<ST>(&s.kr[t][d]) * ks;
                                aq += ld1<ST>(&s.ql[t][d]) * ks;
                            }
                        }
                        sa[t][sx] = (sx < t) ? ak : 0.f;
                        paq[it] = aq;
                        if (oAqkT) st1<ST>(oAqkT + cCC + (size_t)sx * C + t, aq);
                    }
                }
            }
            __syncthreads();   // raw q, k are read above and overwritten by pass A
        }

        // pass A: row threads (t, EPV channels).  K_l = K e^{a}, Q_l = Q e^{a},
        // K_r = K e^{b} (anchored chunks; raw K otherwise), Qp = Q_l e^{gamma_{16i-1}},
        // Kb = K_r e^{G - gamma_{16i+15}}.  Every LDS operand is read as 16-byte
        // vectors up front; the factor of the first / last block (1) is the
        // table's ones row, so that no load sits behind a branch and no product
        // behind a select.
        {
            constexpr int VPR = D / EPV, NV = C * VPR;
            auto ld_row = [](const float* p, float* x) __attribute__((always_inline)) {
#pragma unroll
                for (int q4 = 0; q4 < EPV / 4; ++q4) {
                    const float4 v4 = *reinterpret_cast<const float4*>(p + 4 * q4);
                    x[4 * q4] = v4.x; x[4 * q4 + 1] = v4.y; x[4 * q4 + 2] = v4.z; x[4 * q4 + 3] = v4.w;
                }
            };
            for (int vv = tid; vv < NV; vv += NTH) {
                const int t = vv / VPR, c0 = (vv - t * VPR) * EPV, blk = t / BS;
                const Vec16<ST> qv{*reinterpret_cast<const uint4*>(&s.ql[t][c0])};
                const Vec16<ST> kv{*reinterpret_cast<const uint4*>(&s.kr[t][c0])};
                float at[EPV], te[EPV], fp[EPV], fq[EPV];
                ld_row(&s.g[t][c0], at);
                ld_row(&s.g[BS * blk + BS - 1][c0], te);
                ld_row(&s.fac[blk > 0 ? FAC_EP + blk - 1 : FAC_ONE][c0], fp);
                ld_row(&s.fac[blk < NB - 1 ? FAC_EQ + blk : FAC_ONE][c0], fq);
                float okl[EPV], oql[EPV], okr[EPV], oqp[EPV], okb[EPV];
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    const float bt = te[e] - at[e];
                    const float el = kexp<PREC>(at[e]);
                    const float qf = qv.get(e), kf = kv.get(e);
                    okl[e] = kf * el;
                    oql[e] = qf * el;
                    okr[e] = unsafe ? kf : kf * kexp<PREC>(bt);
                    oqp[e] = oql[e] * fp[e];   // the ones row for the first block
                    okb[e] = okr[e] * fq[e];   // ... and for the last
                }
                if (unsafe && oKb) {
#pragma unroll
                    for (int e = 0; e < EPV; ++e) {
                        float gsfx = te[e] - at[e];   // G - gamma_t
                        for (int m = blk + 1; m < NB; ++m) gsfx += s.g[BS * m + BS - 1][c0 + e];
                        okb[e] = kv.get(e) * kexp<PREC>(gsfx);
                    }
                }
                store_vec<ST>(&s.kl[t][c0], okl);
                store_vec<ST>(&s.ql[t][c0], oql);
                store_vec<ST>(&s.kr[t][c0], okr);
                if (oQp) store_vec<ST>(oQp + cCD + (size_t)t * D + c0, oqp);
                if (oKb) store_vec<ST>(oKb + cCD + (size_t)t * D + c0, okb);
            }
        }
        __syncthreads();
        // PHASE 3

        // pass B: the transposed copies KbT = (K_r diag(e^{G - gamma_{16i+15}}))^T and
        // QpT = (Q_l diag(e^{gamma_{16i-1}}))^T.  Anchored chunks, bf16: per 16 x 16
        // tile (token block i, channel block j) one MFMA forms X diag(s), which leaves
        // channel d of the tile in lane d % 16 with four consecutive tokens per lane
        // -- the transposed layout -- written as 8-byte pieces of KbT / QpT rows.
        // X = K_r or Q_l is exact in bf16; the scale s is split into bf16 hi + lo
        // halves of one K = 32 step, so the product keeps fp32 accuracy until the
        // final rounding.
        if (std::is_same<ST, uint16_t>::value && !unsafe) {
            // wave w: tiles w, w + NW, ... of each output (NB NT / NW per wave),
            // unrolled so that all of a wave's operand reads share one LDS round trip
            constexpr int PBT = NB * NT / NW;
#pragma unroll
            for (int o = 0; o < 2; ++o) {
                ST* out = o ? oQpT : oKbT;
                if (out == nullptr) continue;
                const ST* X = o ? &s.ql[0][0] : &s.kr[0][0];
                Frag4 A[PBT];
                float sv[PBT];
#pragma unroll
                for (int it = 0; it < PBT; ++it) {
                    const int tt = w + NW * it, i = tt / NT, j = tt - i * NT;
                    A[it] = ldfrag4<1, ST>(X, LDK, BS * i, BS * j);
                    sv[it] = o ? fac_ep(s, i, BS * j + r16) : fac_eq(s, i, BS * j + r16);
                }
#pragma unroll
                for (int it = 0; it < PBT; ++it) {
                    const int tt = w + NW * it, i = tt / NT, j = tt - i * NT;
                    const short hi = (short)f2bf(sv[it]), lo = (short)f2bf(sv[it] - bf2f((uint16_t)hi));
                    short4v bh, bl;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool dg = 4 * g4 + e == r16;   // B[k][n] = s[n] on the diagonal
                        bh[e] = dg ? hi : (short)0;
                        bl[e] = dg ? lo : (short)0;
                    }
                    const f32x4 c =
                        __builtin_amdgcn_mfma_f32_16x16x32_bf16(cat4(A[it].h, A[it].h), cat4(bh, bl), zero4(), 0, 0, 0);
                    *reinterpret_cast<uint2*>(out + cCD + (size_t)(BS * j + r16) * C + BS * i + 4 * g4) =
                        make_uint2(pack2bf(c[0], c[1]), pack2bf(c[2], c[3]));
                }
            }
        } else {
            // column threads (d, EPV tokens)
            constexpr int GPC = C / EPV, NV = D * GPC;
            for (int vv = tid; vv < NV; vv += NTH) {
                const int d = vv / GPC, tb = (vv - d * GPC) * EPV;
                float okb[EPV], oqp[EPV];
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    const int t = tb + e, blk = t / BS;
                    const float kr = ld1<ST>(&s.kr[t][d]);
                    if (unsafe) {
                        float gsfx = s.g[BS * blk + BS - 1][d] - s.g[t][d];   // G - gamma_t
                        for (int m = blk + 1; m < NB; ++m) gsfx += s.g[BS * m + BS - 1][d];
                        okb[e] = kr * kexp<PREC>(gsfx);
                    } else {
                        okb[e] = kr * fac_eq(s, blk, d);
                    }
                    oqp[e] = ld1<ST>(&s.ql[t][d]) * fac_ep(s, blk, d);
                }
                if (oKbT) store_vec<ST>(oKbT + cCD + (size_t)d * C + tb, okb);
                if (oQpT) store_vec<ST>(oQpT + cCD + (size_t)d * C + tb, oqp);
            }
        }
        if constexpr (G::STAGE_V) tv.store(&svbuf[0][0], LDK);   // first read by the forward substitution
        __syncthreads();
        // PHASE 4

        // Aqk is staged row-major for coalesced stores; AqkT is written from the
        // accumulators (a lane's four rows of one column are four consecutive AqkT
        // elements)
        ST* stA = G::STG_IN_G ? reinterpret_cast<ST*>(&s.g[0][0]) : &stgbuf[0][0];
        // Split A operands of the solve (bf16 hi, lo of each fp32 value; rows of
        // 16 hi | 16 lo | pad), formed once per chunk by the waves that form or
        // invert the blocks and read by every wave as fragments: the diagonal-block inverses over their own fp32 rows in tii
        // (the same bytes per block), the six off-diagonal blocks -beta A_kk in
        // the g region behind the A_qk staging.  Where that does not fit, each
        // wave splits its own operands.
        constexpr int SPR = 2 * BS + 8, SPB = BS * SPR;
        constexpr int STGB = G::STG_IN_G ? C * LDT * (int)sizeof(ST) : 0;
        constexpr bool SPL = (int)sizeof(tii[0]) == SPB * 2 && STGB + 6 * SPB * 2 <= (int)sizeof(s.g);
        uint16_t* spl = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(&s.g[0][0]) + STGB);
        // lane (r, g) puts / gets A[r][4 g .. 4 g + 3] of a split block
        auto put_split = [&](uint16_t* b, const float* v) __attribute__((always_inline)) {
            const uint32_t h0 = pack2bf(v[0], v[1]), h1 = pack2bf(v[2], v[3]);
            *reinterpret_cast<uint2*>(b + r16 * SPR + 4 * g4) = make_uint2(h0, h1);
            *reinterpret_cast<uint2*>(b + r16 * SPR + BS + 4 * g4) =
                make_uint2(pack2bf_rest(v[0], v[1], h0), pack2bf_rest(v[2], v[3], h1));
        };
        auto get_split = [&](const uint16_t* b) __attribute__((always_inline)) {
            Frag4 f;
            f.h = __builtin_bit_cast(short4v, *reinterpret_cast<const uint2*>(b + r16 * SPR + 4 * g4));
            f.l = __builtin_bit_cast(short4v, *reinterpret_cast<const uint2*>(b + r16 * SPR + BS + 4 * g4));
            return f;
        };
        // the diagonal block's inverse (wave w < NB, block w) and, with SPL, its
        // split rows over its fp32 rows: the wave reads back what its lanes wrote
        // (in order within the wave), then overwrites
        auto invert_block = [&]() __attribute__((always_inline)) {
            diag_inverse_reg<LDA>(&sa[0][0], s.beta, tii);
            if constexpr (SPL) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                const float4 x = *reinterpret_cast<const float4*>(&tii[w][r16][4 * g4]);
                if (a_Tii)
                    *reinterpret_cast<float4*>(a_Tii + (size_t)ch * NB * BS * BS + w * BS * BS + r16 * BS + 4 * g4) = x;
                const float v4[4] = {x.x, x.y, x.z, x.w};
                put_split(reinterpret_cast<uint16_t*>(&tii[w][0][0]), v4);
            }
        };
        // the solve's off-diagonal A operand -beta_t A_kk[t][s] of block pair (i, j),
        // i > j, split once instead of in every wave
        auto split_pair = [&](int i, int j) __attribute__((always_inline)) {
            const float4 x = *reinterpret_cast<const float4*>(&sa[BS * i + r16][BS * j + 4 * g4]);
            const float br = -s.beta[BS * i + r16];
            const float lv[4] = {br * x.x, br * x.y, br * x.z, br * x.w};
            put_split(spl + (i * (i - 1) / 2 + j) * SPB, lv);
        };
        // With eight waves and the split operands, waves 0-3 form the diagonal
        // tiles and invert them at once (their own LDS writes, no barrier) while
        // waves 4-7 form the six off-diagonal tiles and split them: the inverses
        // run beside the products instead of after them.
        constexpr bool EARLY = SPL && NW == 2 * NB;
        constexpr int OFFD[6] = {1, 3, 4, 6, 7, 8};   // tile_ij indices of the blocks below the diagonal
        if (!unsafe) {
            // 10 lower sub-block tiles of Akk and Aqk; the B operand is shared: K_r of
            // block j times the tile's channel factor (F_ij, 1 between adjacent
            // blocks, e^{-T_i} on the diagonal).  Diagonal tiles of blocks in pmask
            // were formed pair by pair.
            auto form_tile = [&](int i, int j) __attribute__((always_inline)) {
                const float* fsc = &s.fac[(j == i) ? FAC_FD + i : (j == i - 1) ? 0 : fac_f_row(i, j)][0];
                f32x4 P = zero4(), Q = zero4();
                // both operands are rows of LDS tiles: contiguous k-slots, one
                // 16-byte read per lane and operand
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    const Frag8 Ak = ldfrag_c<PREC, ST>(&s.kl[0][0], LDK, BS * i, 32 * ks);
                    const Frag8 Aq = ldfrag_c<PREC, ST>(&s.ql[0][0], LDK, BS * i, 32 * ks);
                    const Frag8 Bk = (j == i - 1) ? ldfrag_c<PREC, ST>(&s.kr[0][0], LDK, BS * j, 32 * ks)
                                                  : ldfrag_c_scaled<PREC, ST>(&s.kr[0][0], LDK, BS * j, 32 * ks,
                                                                              fsc + 32 * ks);
                    P = mma<PREC>(Ak, Bk, P);
                    Q = mma<PREC>(Aq, Bk, Q);
                }
                float aq[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * i + 4 * g4 + e, sx = BS * j + r16;
                    sa[t][sx] = (sx < t) ? P[e] : 0.f;
                    aq[e] = (sx <= t) ? Q[e] : 0.f;
                    if (oAqk) st1<ST>(stA + t * LDT + sx, aq[e]);
                }
                if (oAqkT) st4(oAqkT + cCC + (size_t)(BS * j + r16) * C + BS * i + 4 * g4, aq);
            };
            if constexpr (EARLY) {
                if (w < NB) {
                    if (!((pmask >> w) & 1)) form_tile(w, w);
                } else {
                    for (int o = w - NB; o < 6; o += NW - NB) {
                        int i, j;
                        tile_ij(OFFD[o], i, j);
                        form_tile(i, j);
                    }
                }
            } else {
                for (int tix = w; tix < 10; tix += NW) {
                    int i, j;
                    tile_ij(tix, i, j);
                    if (j == i && ((pmask >> i) & 1)) continue;
                    form_tile(i, j);
                }
            }
            // the diagonal entries of A_qk formed in phase 2, from registers
            if (oAqk && (((pmask & ~qmask) >> w) & 1)) {
#pragma unroll
                for (int e = 0; e < 4; ++e) st1<ST>(stA + (BS * w + 4 * g4 + e) * LDT + BS * w + r16, saq[e]);
            }
            if (oAqk && qmask) {
                const int nent = __popc(qmask) * BS * BS;
#pragma unroll
                for (int it = 0; it < NPW; ++it) {
                    const int pp = tid + NTH * it;
                    if (pp < nent) {
                        const int kb = pp / (BS * BS), e = pp - kb * BS * BS;
                        int blk = 0;
                        for (int m = qmask, c = 0;; m &= m - 1, ++c)
                            if (c == kb) { blk = __ffs(m) - 1; break; }
                        st1<ST>(stA + (BS * blk + e / BS) * LDT + BS * blk + e % BS, paq[it]);
                    }
                }
            }
            // strictly upper sub-block tiles are zero
            for (int idx = tid; idx < 6 * BS * BS; idx += NTH) {
                const int tile = idx / (BS * BS), e = idx - tile * BS * BS;
                const int i = (tile < 3) ? 0 : (tile < 5) ? 1 : 2;
                const int j = (tile < 3) ? tile + 1 : (tile < 5) ? tile - 1 : 3;
                const int t = BS * i + e / BS, sx = BS * j + (e % BS);
                sa[t][sx] = 0.f;
                if (oAqk) st1<ST>(stA + t * LDT + sx, 0.f);
            }
            constexpr int ZW = 10 % NW;   // waves >= ZW formed one tile fewer of the ten
            if (oAqkT && w >= ZW) {
                // they write the six zero tiles
                const float z[4] = {0.f, 0.f, 0.f, 0.f};
                for (int u = w - ZW; u < 6; u += NW - ZW) {   // tile (i, j), i < j
                    const int i = (u < 3) ? 0 : (u < 5) ? 1 : 2;
                    const int j = (u < 3) ? u + 1 : (u < 5) ? u - 1 : 3;
                    st4(oAqkT + cCC + (size_t)(BS * j + r16) * C + BS * i + 4 * g4, z);
                }
            }
        }
        if constexpr (EARLY) {
            // the wave's own tiles (unsafe chunks: A_kk formed pair by pair above)
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (w < NB) {
                invert_block();
            } else {
                for (int o = w - NB; o < 6; o += NW - NB) {
                    int i, j;
                    tile_ij(OFFD[o], i, j);
                    split_pair(i, j);
                }
            }
        }
        __syncthreads();
        // PHASE 5
        if (!unsafe) {
            if (oAqk) tile_out<ST, C, C, NTH>(stA, LDT, oAqk + cCC, C, C);
            if (a_Akk) tile_out<float, C, C, NTH>(&sa[0][0], LDA, a_Akk + cCC, C, C);
        }
        if constexpr (!EARLY) {
            if (w < NB) invert_block();
            if constexpr (SPL) {
                constexpr int LW0 = (NW > NB) ? NB : 0, LWN = NW - LW0;
                if (w >= LW0)
                    for (int p = w - LW0; p < 6; p += LWN) {
                        const int i = (p < 1) ? 1 : (p < 3) ? 2 : 3;
                        split_pair(i, p - i * (i - 1) / 2);
                    }
            }
            __syncthreads();
        }
        // PHASE 6
        if (!SPL && a_Tii && tid < NB * BS * BS / 4) {
            const int i = tid / (BS * BS / 4), e4 = (tid - i * (BS * BS / 4)) * 4;
            *reinterpret_cast<float4*>(a_Tii + (size_t)ch * NB * BS * BS + i * BS * BS + e4) =
                *reinterpret_cast<const float4*>(&tii[i][e4 / BS][e4 % BS]);
        }

        // block forward substitution; the wave's column tiles of [Kt | beta V] advance together
        f32x4 X[TPW][NB];
        Frag4 XB[TPW][NB - 1];   // X's split-bf16 B fragments, formed once for the later blocks
        bool tok[TPW], isK[TPW];
        int dcol[TPW];
#pragma unroll
        for (int jj = 0; jj < TPW; ++jj) {
            const int ct = w + NW * jj;
            tok[jj] = ct < NCT;
            isK[jj] = ct < NT;
            dcol[jj] = (isK[jj] ? ct : ct - NT) * BS + r16;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            f32x4 Y[TPW];
            // right-hand sides, rows t = 16 i + 4 g4 + e of column d: bf16 columns by
            // transposing reads, beta of the lane's four rows as one vector
            const float4 b4 = *reinterpret_cast<const float4*>(&s.beta[BS * i + 4 * g4]);
            const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int jj = 0; jj < TPW; ++jj) {
                const int d = dcol[jj];
                float col[4] = {0.f, 0.f, 0.f, 0.f};
                float fe = 1.f;
                if constexpr (std::is_same<ST, uint16_t>::value) {
                    if (tok[jj]) {
                        const int ct = d - r16;
                        if (isK[jj]) ld_col4(&s.kl[0][0], LDK, ct, BS * i, col);
                        else if constexpr (G::STAGE_V) ld_col4(&svbuf[0][0], LDK, ct, BS * i, col);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = BS * i + 4 * g4 + e;
                        if (tok[jj]) {
                            if (isK[jj]) col[e] = ld1<ST>(&s.kl[t][d]);
                            else if constexpr (G::STAGE_V) col[e] = ld1<ST>(&svbuf[t][d]);
                        }
                    }
                }
                if (tok[jj] && isK[jj]) fe = fac_ep(s, i, d);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = BS * i + 4 * g4 + e;
                    float rv = 0.f;
                    if (tok[jj]) {
                        if (isK[jj]) {
                            rv = bv[e] * fe * col[e];
                        } else if constexpr (G::STAGE_V) {
                            rv = bv[e] * col[e];
                        } else {
                            rv = (t < valid && d < dio) ? bv[e] * ld1<ST>(v + base + (size_t)t * rs + d) : 0.f;
                        }
                    }
                    Y[jj][e] = rv;
                }
            }
            const float brow = -s.beta[BS * i + r16];
#pragma unroll
            for (int j = 0; j < i; ++j) {
                Frag4 A;
                if constexpr (SPL) {
                    A = get_split(spl + (i * (i - 1) / 2 + j) * SPB);
                } else {
                    const float4 x = *reinterpret_cast<const float4*>(&sa[BS * i + r16][BS * j + 4 * g4]);
                    const float lv[4] = {brow * x.x, brow * x.y, brow * x.z, brow * x.w};
                    A = frag4_from_f32<3>(lv);
                }
#pragma unroll
                for (int jj = 0; jj < TPW; ++jj)
                    if (tok[jj]) Y[jj] = mma4f<3>(A, XB[jj][j], Y[jj]);
            }
            const Frag4 Tf = SPL ? get_split(reinterpret_cast<const uint16_t*>(&tii[i][0][0]))
                                 : ldfrag4<3, float>(&tii[i][0][0], BS + 4, 0, 0);
#pragma unroll
            for (int jj = 0; jj < TPW; ++jj) {
                X[jj][i] = tok[jj] ? mma4f<3>(Tf, accfrag4<3>(Y[jj]), zero4()) : zero4();
                if (i < NB - 1) XB[jj][i] = accfrag4<3>(X[jj][i]);
            }
        }
        __syncthreads();
        // PHASE 7
        // staging: W -> kl region, U -> ql region (both dead now); WT straight from
        // the accumulators (four consecutive tokens of one channel per lane)
        ST* stW = &s.kl[0][0];
        ST* stU = &s.ql[0][0];
#pragma unroll
        for (int jj = 0; jj < TPW; ++jj)
            if (tok[jj])
#pragma unroll
                for (int i = 0; i < NB; ++i) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = BS * i + 4 * g4 + e, d = dcol[jj];
                        st1<ST>((isK[jj] ? stW : stU) + t * LDK + d, X[jj][i][e]);
                    }
                    if (isK[jj] && oWT) {
                        const float x[4] = {X[jj][i][0], X[jj][i][1], X[jj][i][2], X[jj][i][3]};
                        st4(oWT + cCD + (size_t)dcol[jj] * C + BS * i + 4 * g4, x);
                    }
                }
        __syncthreads();
        tile_out<ST, C, D, NTH>(stW, LDK, oW + cCD, D, C);
        tile_out<ST, C, D, NTH>(stU, LDK, oU + cCD, D, C);
        // PHASE 8
    };
    if (dfl & 31)
        tail(std::true_type{});
    else
        tail(std::false_type{});
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
#ifndef KDA_PREP_NTH
#define KDA_PREP_NTH 512
#endif
template <int D, typename ST, typename TG>
static hipError_t launch_prep_t(const PrepArgs& a, int nchunks, hipStream_t st) {
    constexpr int PREC = std::is_same<ST, float>::value ? 3 : 1;
    // eight waves per chunk where the registers allow four waves per SIMD;
    // bf16 at D = 128 (133 KB of LDS: one workgroup per CU, 123 VGPRs) sixteen,
    // four per SIMD on one chunk: config 3's prep 396 -> 368 us, bit-identical
    constexpr int NTH = (D >= 128 && std::is_same<ST, uint16_t>::value) ? 1024 : (D >= 64) ? KDA_PREP_NTH : 256;
    hipLaunchKernelGGL((kda_prep_kernel<D, ST, TG, PREC, NTH>), dim3(nchunks), dim3(NTH), 0, st, a);
    return hipGetLastError();
}

// g_kind: 0 fp32 g, 1 bf16 g, 2 one fp32 decay per (b, t, h) (bf16 inputs at
// D <= 64 only)
hipError_t launch_prep(const PrepArgs& a, int D, int in_bf16, int g_kind, int nchunks, hipStream_t st) {
    if (g_kind == 2) {
        if (!in_bf16) return hipErrorInvalidValue;
        if (D == 32) return launch_prep_t<32, uint16_t, GHead>(a, nchunks, st);
        if (D == 64) return launch_prep_t<64, uint16_t, GHead>(a, nchunks, st);
        return hipErrorInvalidValue;
    }
    const int g_bf16 = g_kind == 1;
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

}  // namespace kda
