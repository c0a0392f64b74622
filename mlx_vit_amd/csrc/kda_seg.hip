// kda_seg.hip -- the bf16 forward recurrence at D = 128 split over segments of
// the sequence, so that a few long (batch, head) sequences fill the GPU.
//
// A segment of L chunks maps its start state to its end state affinely (the
// state orientation inside the kernels is Sigma = S^T, [dk][dv]):
//     Sigma_out = M Sigma_in + X,
// X the end state of the segment's chunk loop from Sigma = 0, and M (dk x dk)
// the product of the chunks' transitions diag(e^G) - Kb^T W, i.e. the chunk
// loop with U = 0 run on the D identity columns.  Three launches:
//   kda_segchain_kernel<D, 1>  pass A: X and M of every segment but the last,
//                              one workgroup per (b, h, segment);
//   kda_segscan_kernel<D>      pass B: Sigma_in of segments 1 .. nseg-1 in
//                              order, per (b, h) and 16-column block;
//   kda_segchain_kernel<D, 0>  pass C: every segment's forward from its
//                              Sigma_in -- O, and the final state from the
//                              last segment;
//   kda_segchain_kernel<D, 2>  pass C of the backward's state recompute: the
//                              chunk-start states h and V' = U - W h of every
//                              chunk instead of O (after passes A and B).
// This is the chunk loop of nope_gdn_mlx.py:2408-2451 (V' = U - W Sigma, O =
// Qp Sigma + Aqk V', Sigma <- diag(e^G) Sigma + Kb^T V') regrouped: the loop is
// linear in Sigma, so its segments compose.
//
// Waves own state columns and never exchange anything: wave w keeps all D rows
// of its columns of Sigma in fp32 accumulators, so V' = U - W Sigma, O and the
// state update of those columns take their B operands from the wave's own
// registers, with the chunk's A operands (W, Qp, Kb^T, Aqk) read from LDS.
// Pass C: wave w of 8 owns dv columns 16 w .. 16 w + 15; pass A: waves 0-3 own
// 32 dv columns each (X), waves 4-7 32 identity columns each (M).  The chunk's
// slabs arrive by LDS DMA into NS sets, one chunk (pass C) or two (pass A) ahead.
//
// Row order.  Inside these kernels the state's dk index and the chunk's token
// index run in the order perm_row (below): accumulator row rho = 16 a + 4 g + e
// (16-row tile a, lane group g, element e) holds index
//     pi(rho) = 32 (a >> 1) + 4 (a & 1) + 8 g + e.
// The B operand of k-step s is the accumulator pair (tiles 2 s, 2 s + 1), which
// gives lane group g the indices 32 s + 8 g .. + 7 -- contiguous -- so every A
// fragment is one 16-byte LDS read per lane at its row pi(rho), and the
// tiles' row swizzle (SwzG) puts the rows read together on distinct banks.
// Only addresses change: states are loaded and stored, and O rows written, at
// their natural indices.
#include "kda_internal.h"

namespace kda {

namespace {

__device__ __forceinline__ int perm_row(int rho) {
    return 32 * (rho >> 5) + 4 * ((rho >> 4) & 1) + 8 * ((rho >> 2) & 3) + (rho & 3);
}

// Swizzle of the DMA'd tiles for row-gathered reads: the 16-byte chunk c of
// row r lies at chunk c ^ f(r).  The rows that 8 (16) consecutive lanes read
// are r = B + 8 u + v, v < 4, u < 2 (4); f maps them to distinct chunks.
template <int RB>
struct SwzG {
    static constexpr int NCH = RB / 16;
    static_assert(NCH == 8 || NCH == 16, "rows of 128 or 256 bytes");
    __device__ __forceinline__ static int f(int r) { return (r & 3) | (((r >> 3) & (NCH / 8 == 2 ? 3 : 1)) << 2); }
    __device__ __forceinline__ static int at(int r, int b) { return r * RB + (((b >> 4) ^ f(r)) << 4) + (b & 15); }
};

// DmaTile with the SwzG swizzle: an NR x RB-byte tile in 1 KB wave-instructions,
// wave `first` of STEP issuing instructions first, first + STEP, ...
template <int NR, int RB, int STEP>
struct DmaTileG {
    static constexpr int NI = NR * RB / 1024, COUNT = NI / STEP;
    static_assert((NR * RB) % 1024 == 0 && NI % STEP == 0, "whole 1 KB blocks per wave");
    __device__ __forceinline__ static void offsets(uint32_t (&off)[COUNT], size_t GS, int first, int lane) {
#pragma unroll
        for (int k = 0; k < COUNT; ++k) {
            const int i = first + STEP * k;
            const int p = 1024 * i + 16 * lane, r = p / RB, pc = (p % RB) >> 4;
            off[k] = (uint32_t)(r * GS) + ((uint32_t)(pc ^ SwzG<RB>::f(r)) << 4);
        }
    }
    __device__ __forceinline__ static void issue_s(const char* g, const uint32_t (&off)[COUNT], char* lds, int first) {
#pragma unroll
        for (int k = 0; k < COUNT; ++k) dma16_s(g, off[k], lds + 1024 * (first + STEP * k));
    }
};

// A fragment, k-slots 8 g .. 8 g + 7 = k0 + 8 g .. + 7 of row `row`: one 16-byte read
template <int RB>
__device__ __forceinline__ bf16x8 afrag(const uint16_t* M, int row, int k0) {
    const int g = lane_id() >> 4;
    return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(M) + SwzG<RB>::at(row, 2 * (k0 + 8 * g)));
}

// rows r0 + 8 g + e, e = 0..3, of column n0 + (lane % 16): the accumulator
// layout of a row-permuted 16-row block, by one transposing read per lane
template <int RB>
__device__ __forceinline__ f32x4 col4g(const uint16_t* M, int n0, int r0) {
    const int l = lane_id(), j = l & 15, g = l >> 4;
    const short4v x = ld_tr4(reinterpret_cast<const uint16_t*>(
        reinterpret_cast<const char*>(M) + SwzG<RB>::at(r0 + 8 * g + (j >> 2), 2 * (n0 + 4 * (j & 3)))));
    return f32x4{bf2f((uint16_t)x[0]), bf2f((uint16_t)x[1]), bf2f((uint16_t)x[2]), bf2f((uint16_t)x[3])};
}

// B fragment of k-step s from the accumulator pair (tiles 2 s, 2 s + 1), bf16
__device__ __forceinline__ bf16x8 bfrag(const f32x4& lo, const f32x4& hi) {
    return __builtin_bit_cast(bf16x8, make_uint4(pack2bf(lo[0], lo[1]), pack2bf(lo[2], lo[3]),
                                                 pack2bf(hi[0], hi[1]), pack2bf(hi[2], hi[3])));
}

__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Lane (g, r) of a 16x16 accumulator holds x[e] = X[4 g + e][r].  Returns y
// with y[c] = X[4 g + (r & 3)][4 (r >> 2) + c]: four consecutive columns of one
// row, for one 8-byte store.  A 4x4 transpose inside each quad of lanes: in
// round k the lane sends its element (p + k) & 3 (p = r & 3) and receives,
// from quad lane (p - k) & 3, that lane's element p.
__device__ __forceinline__ f32x4 quad_transpose(const f32x4& x) {
    const int p = lane_id() & 3;
    auto pick = [&](int i) __attribute__((always_inline)) {
        return (i == 0) ? x[0] : (i == 1) ? x[1] : (i == 2) ? x[2] : x[3];
    };
    f32x4 y;
    y[0] = (p == 0) ? x[0] : 0.f;
    y[1] = (p == 1) ? x[1] : 0.f;
    y[2] = (p == 2) ? x[2] : 0.f;
    y[3] = (p == 3) ? x[3] : 0.f;
    // quad_perm controls: destination p reads quad lane (p - k) & 3
#pragma unroll
    for (int k = 1; k < 4; ++k) {
        const float z = pick((p + k) & 3);
        float v;
        if (k == 1) v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(z), 0x93, 0xf, 0xf, false));
        else if (k == 2) v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(z), 0x4E, 0xf, 0xf, false));
        else v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(z), 0x39, 0xf, 0xf, false));
        const int s = (p - k) & 3;
        if (s == 0) y[0] = v;
        if (s == 1) y[1] = v;
        if (s == 2) y[2] = v;
        if (s == 3) y[3] = v;
    }
    return y;
}

template <int D, int PASS, int NW>
struct SegLayout {
    static constexpr int NS = PASS == 0 ? 2 : 3;                   // LDS sets (PASS 2: no Qp, Aqk)
    static constexpr int RB_W = 2 * D, RB_C = 2 * C;              // swizzled row bytes
    static constexpr int W_OFF = 0;                               // W   [C][D]
    static constexpr int U_OFF = W_OFF + C * RB_W;                // U   [C][D]
    static constexpr int KBT_OFF = U_OFF + C * RB_W;              // Kb^T [D][C]
    static constexpr int QP_OFF = KBT_OFF + D * RB_C;             // Qp  [C][D]  (pass C)
    static constexpr int AQK_OFF = QP_OFF + (PASS == 0 ? C * RB_W : 0);   // Aqk [C][C] (pass C)
    static constexpr int EG_OFF = AQK_OFF + (PASS == 0 ? C * RB_C : 0);   // e^G [D] fp32
    static constexpr int SET_BYTES = (EG_OFF + 4 * D + 1023) & ~1023;
    static constexpr int BYTES = NS * SET_BYTES;
    static_assert(BYTES <= 160 * 1024, "segment chain LDS");
    using TW = DmaTileG<C, RB_W, NW>;
    using TK = DmaTileG<D, RB_C, NW>;
    using TA = DmaTileG<C, RB_C, NW>;
    static constexpr int EG_LANES = 4 * D / 16 / NW;              // 16-byte lanes of e^G per wave
    // DMA wave-instructions per wave per chunk (W, U, Kb^T [, Qp, Aqk], e^G)
    static constexpr int LI = 2 * TW::COUNT + TK::COUNT + (PASS == 0 ? TW::COUNT + TA::COUNT : 0) + 1;
};

}  // namespace

// Pass C (PASS 0): the forward of one segment from its start state.  Pass A
// (PASS 1): the segment's map (X, M).  PASS 2: the segment's chunk-start
// states h and V' = U - W h (bf16, natural indices: h[chunk][dk][dv],
// V'[chunk][t][dv]) from its start state, for the backward.  One 512-thread
// workgroup per (b, h, segment); layout, roles and row order in the file
// comment.
template <int D, int PASS, int NW>
__global__ __launch_bounds__(64 * NW) void kda_segchain_kernel(const SegArgs a) {
    using ST = uint16_t;
    using Lay = SegLayout<D, PASS, NW>;
    using TW = typename Lay::TW;
    using TK = typename Lay::TK;
    using TA = typename Lay::TA;
    constexpr int NS = Lay::NS, NI = D / BS, KS = D / 32, NJ = (PASS == 1) ? 2 * D / (16 * NW) : D / (16 * NW);
    constexpr int RB_W = Lay::RB_W, RB_C = Lay::RB_C, LI = Lay::LI;
    static_assert(NJ >= 1 && NS >= 2 && Lay::EG_LANES >= 1, "whole column tiles per wave");
    __shared__ __align__(1024) char smem[Lay::BYTES];

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15,
              g4 = l >> 4;
    __builtin_assume(w >= 0 && w < NW);
    // segments this pass covers (pass A: the last one only for the reverse scan)
    const int nsegw = (PASS == 1 && !a.all_maps) ? a.nseg - 1 : a.nseg;
    const int bh = blockIdx.x / nsegw, seg = blockIdx.x - bh * nsegw;
    const int b = bh / a.H, h = bh - b * a.H;
    const int n0 = seg * a.seg_len, L = min(a.nc, n0 + a.seg_len) - n0;
    constexpr int CPW = BS * NJ;                                        // columns per wave
    const bool ident = PASS == 1 && w >= NW / 2;                        // identity columns (M)
    const int cb = (PASS == 1) ? CPW * (w % (NW / 2)) : CPW * w;        // first owned column
    const size_t seg_ix = (size_t)bh * a.nseg + seg;

    // ---- the start state of the owned columns (rows in perm_row order) ----
    f32x4 S[NI][NJ];
    {
        // this (b, h)'s start state: s0 for the first segment, pass B's result after
        const float* src = nullptr;
        if constexpr (PASS != 1)
            src = (seg == 0) ? (a.s0 ? a.s0 + (size_t)bh * D * D : nullptr) : a.segS + seg_ix * D * D;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int col = cb + BS * j + r16, row0 = perm_row(BS * i + 4 * g4);
                if constexpr (PASS != 1) {
                    S[i][j] = zero4();
                    if (src) {
                        const float4 x = *reinterpret_cast<const float4*>(src + (size_t)col * D + row0);
                        S[i][j] = f32x4{x.x, x.y, x.z, x.w};
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) S[i][j][e] = (ident && row0 + e == col) ? 1.f : 0.f;
                }
            }
    }

    // ---- LDS DMA of a chunk's slabs into a set ----
    const char* gW = static_cast<const char*>(a.W);
    const char* gU = static_cast<const char*>(a.U);
    const char* gKbT = static_cast<const char*>(a.KbT);
    const char* gQp = static_cast<const char*>(a.Qp);
    const char* gAqk = static_cast<const char*>(a.Aqk);
    const char* gEg = reinterpret_cast<const char*>(a.eG);
    uint32_t oW[TW::COUNT], oK[TK::COUNT], oA[TA::COUNT];
    TW::offsets(oW, RB_W, w, l);
    TK::offsets(oK, RB_C, w, l);
    TA::offsets(oA, RB_C, w, l);
    // e^G: 4 D bytes, EG_LANES 16-byte lanes per wave
    constexpr int EGW = 16 * Lay::EG_LANES;
    const uint32_t oE = (uint32_t)(EGW * w + 16 * (l < Lay::EG_LANES ? l : 0));
    auto dma_chunk = [&](int c, char* sb) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * a.nc + c;
        TW::issue_s(gW + ch * C * D * 2, oW, sb + Lay::W_OFF, w);
        TW::issue_s(gU + ch * C * D * 2, oW, sb + Lay::U_OFF, w);
        TK::issue_s(gKbT + ch * C * D * 2, oK, sb + Lay::KBT_OFF, w);
        if constexpr (PASS == 0) {
            TW::issue_s(gQp + ch * C * D * 2, oW, sb + Lay::QP_OFF, w);
            TA::issue_s(gAqk + ch * C * C * 2, oA, sb + Lay::AQK_OFF, w);
        }
        if (l < Lay::EG_LANES) dma16_s(gEg + ch * D * 4, oE, sb + Lay::EG_OFF + EGW * w);
    };

    // O of the previous chunk: lane (g, 4 q + p) holds row pi(16 m + 4 g + p),
    // columns 4 q .. 4 q + 3 of its tile (quad_transpose), packed
    uint2 Opk[NB][NJ];
    auto store_o = [&](int c) __attribute__((always_inline)) {
        const int t0 = c * C, valid = min(C, a.T - t0);
        ST* op = static_cast<ST*>(a.o) + (((size_t)b * a.T + t0) * a.H + h) * D;
        const size_t rs = (size_t)a.H * D;
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int row = perm_row(BS * m + 4 * g4) + (r16 & 3), col = cb + BS * j + 4 * (r16 >> 2);
                if (row < valid) *reinterpret_cast<uint2*>(op + row * rs + col) = Opk[m][j];
            }
    };

    // PASS 2: h and V' of the previous chunk, packed the way O is (four
    // consecutive columns of one row per lane)
    uint2 Hpk[NI][NJ], Vpk[NB][NJ];
    auto store_hv = [&](int c) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * a.nc + c;
        ST* hp = static_cast<ST*>(a.h) + ch * D * D;
        ST* vp = static_cast<ST*>(a.Vp) + ch * C * D;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int col = cb + BS * j + 4 * (r16 >> 2);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                *reinterpret_cast<uint2*>(hp + (size_t)(perm_row(BS * i + 4 * g4) + (r16 & 3)) * D + col) = Hpk[i][j];
#pragma unroll
            for (int m = 0; m < NB; ++m)
                *reinterpret_cast<uint2*>(vp + (size_t)(perm_row(BS * m + 4 * g4) + (r16 & 3)) * D + col) = Vpk[m][j];
        }
    };

#pragma unroll
    for (int c = 0; c < NS - 1; ++c)
        if (c < L) dma_chunk(n0 + c, smem + c * Lay::SET_BYTES);

    for (int n = 0; n < L; ++n) {
        // chunk n's DMA done (this wave's share); later chunks may stay in flight
        dma_wait_chunks<LI>(min(L - 1, n + NS - 2) - n);
        lds_barrier();   // every wave's share landed; set (n - 1) % NS is free
        if constexpr (PASS == 0)
            if (n > 0) store_o(n0 + n - 1);
        if constexpr (PASS == 2)
            if (n > 0) store_hv(n0 + n - 1);
        if (n + NS - 1 < L) dma_chunk(n0 + n + NS - 1, smem + ((n + NS - 1) % NS) * Lay::SET_BYTES);
        const char* sb = smem + (n % NS) * Lay::SET_BYTES;
        const ST* sW = reinterpret_cast<const ST*>(sb + Lay::W_OFF);
        const ST* sU = reinterpret_cast<const ST*>(sb + Lay::U_OFF);
        const ST* sKbT = reinterpret_cast<const ST*>(sb + Lay::KBT_OFF);
        const float* sEg = reinterpret_cast<const float*>(sb + Lay::EG_OFF);

        if constexpr (PASS == 2) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const f32x4 y = quad_transpose(S[i][j]);
                    Hpk[i][j] = make_uint2(pack2bf(y[0], y[1]), pack2bf(y[2], y[3]));
                }
        }
        // B operands of the chunk-start state
        bf16x8 Bs[NJ][KS];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int s = 0; s < KS; ++s) Bs[j][s] = bfrag(S[2 * s][j], S[2 * s + 1][j]);
        // V' = U - W Sigma (identity columns: U = 0); token rows pi(16 m + r16)
        f32x4 Vp[NB][NJ];
#pragma unroll
        for (int m = 0; m < NB; ++m) {
            const int row = perm_row(BS * m + r16);
            bf16x8 Aw[KS];
#pragma unroll
            for (int s = 0; s < KS; ++s) Aw[s] = afrag<RB_W>(sW, row, 32 * s);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                f32x4 P = zero4();
#pragma unroll
                for (int s = 0; s < KS; ++s) P = mfma(Aw[s], Bs[j][s], P);
                if (!ident) {
                    const f32x4 u = col4g<RB_W>(sU, cb + BS * j, perm_row(BS * m));
                    Vp[m][j] = f32x4{u[0] - P[0], u[1] - P[1], u[2] - P[2], u[3] - P[3]};
                } else {
                    Vp[m][j] = negacc(P);
                }
            }
        }
        bf16x8 Bv[NJ][2];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int s = 0; s < 2; ++s) Bv[j][s] = bfrag(Vp[2 * s][j], Vp[2 * s + 1][j]);
        if constexpr (PASS == 2) {
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const f32x4 y = quad_transpose(Vp[m][j]);
                    Vpk[m][j] = make_uint2(pack2bf(y[0], y[1]), pack2bf(y[2], y[3]));
                }
        }
        if constexpr (PASS == 0) {
            // O = Qp Sigma + Aqk V' (row block m holds tokens 32 (m >> 1) ..
            // + 31, and Aqk is zero above the diagonal: k-steps s <= m >> 1)
            const ST* sQp = reinterpret_cast<const ST*>(sb + Lay::QP_OFF);
            const ST* sAqk = reinterpret_cast<const ST*>(sb + Lay::AQK_OFF);
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                const int row = perm_row(BS * m + r16);
                bf16x8 Aq[KS], Aa[2];
#pragma unroll
                for (int s = 0; s < KS; ++s) Aq[s] = afrag<RB_W>(sQp, row, 32 * s);
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    if (s <= (m >> 1)) Aa[s] = afrag<RB_C>(sAqk, row, 32 * s);
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    f32x4 O = zero4();
#pragma unroll
                    for (int s = 0; s < KS; ++s) O = mfma(Aq[s], Bs[j][s], O);
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        if (s <= (m >> 1)) O = mfma(Aa[s], Bv[j][s], O);
                    const f32x4 y = quad_transpose(O);
                    Opk[m][j] = make_uint2(pack2bf(y[0], y[1]), pack2bf(y[2], y[3]));
                }
            }
        }
        // Sigma <- diag(e^G) Sigma + Kb^T V'; dk rows pi(16 i + r16)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int row = perm_row(BS * i + r16);
            bf16x8 Ak[2];
#pragma unroll
            for (int s = 0; s < 2; ++s) Ak[s] = afrag<RB_C>(sKbT, row, 32 * s);
            const float4 eg = *reinterpret_cast<const float4*>(sEg + perm_row(BS * i + 4 * g4));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                f32x4 x = f32x4{S[i][j][0] * eg.x, S[i][j][1] * eg.y, S[i][j][2] * eg.z, S[i][j][3] * eg.w};
#pragma unroll
                for (int s = 0; s < 2; ++s) x = mfma(Ak[s], Bv[j][s], x);
                S[i][j] = x;
            }
        }
    }

    if constexpr (PASS == 2) {
        store_hv(n0 + L - 1);
    } else if constexpr (PASS == 0) {
        store_o(n0 + L - 1);
        if (seg == a.nseg - 1 && a.s_final) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + cb + BS * j + r16) * D +
                                               perm_row(BS * i + 4 * g4)) =
                        make_float4(S[i][j][0], S[i][j][1], S[i][j][2], S[i][j][3]);
        }
    } else if (!ident) {
        // X, reference orientation [dv][dk]
        float* X = a.segX + seg_ix * D * D;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                *reinterpret_cast<float4*>(X + (size_t)(cb + BS * j + r16) * D + perm_row(BS * i + 4 * g4)) =
                    make_float4(S[i][j][0], S[i][j][1], S[i][j][2], S[i][j][3]);
    } else {
        // M^T [dk_in][dk_out] as two bf16 planes, hi = bf16(M), lo = bf16(M - hi):
        // this lane's four rows of M are four consecutive dk_out
        ST* Mh = a.segM + seg_ix * 2 * D * D;
        ST* Ml = Mh + (size_t)D * D;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const size_t o = (size_t)(cb + BS * j + r16) * D + perm_row(BS * i + 4 * g4);
                const uint32_t h0 = pack2bf(S[i][j][0], S[i][j][1]), h1 = pack2bf(S[i][j][2], S[i][j][3]);
                *reinterpret_cast<uint2*>(Mh + o) = make_uint2(h0, h1);
                *reinterpret_cast<uint2*>(Ml + o) = make_uint2(pack2bf_rest(S[i][j][0], S[i][j][1], h0),
                                                               pack2bf_rest(S[i][j][2], S[i][j][3], h1));
            }
    }
}

// Pass B (REV = false): Sigma_in of segments 1 .. nseg - 1 of one (b, h), 16 dv
// columns per workgroup, Sigma_in[s + 1] = M_s Sigma_in[s] + X_s with fp32-accurate
// split-bf16 products (Sigma and M as bf16 hi + lo).  Wave w owns the row
// tiles 2 w and 2 w + 1 (dk_out rows 32 w .. 32 w + 31) of the columns: four
// waves share a step's products instead of each forming all 128 rows of its
// own columns.  Those two tiles are the B operand of k-step w of the next
// step, so each wave passes its split fragments lane for lane to the others
// through a double-buffered LDS exchange, one barrier per step.  M_s^T (hi
// and lo planes) reaches LDS by DMA one step ahead and is read once per
// workgroup; X_s is loaded one step ahead into registers; a step's result is
// stored during the next step, so that no wait at a step's start covers a
// store just issued.  Natural row order; written in the reference orientation
// [dv][dk], as s0 is.  Same products in the same order as one wave forming
// all rows: the results do not depend on the split.
// REV = true: the backward's reverse scan, from ds_final through segments
// nseg - 1 .. 1: dSigma_{s-1} = M_s^T dSigma_s + X_rev_s, written to segS[s - 1]
// (the segment's reverse map on dSigma is the transpose of its forward map, so
// the A operand reads the stored M^T planes by rows instead of transposed).
template <int D, bool REV = false>
__global__ __launch_bounds__(256) void kda_segscan_kernel(const SegArgs a) {
    using ST = uint16_t;
    constexpr int NI = D / BS, KS = D / 32, RB = 2 * D, PLANE = D * RB;
    static_assert(NI == 2 * KS && KS == 4, "four waves, wave w owning row tiles 2 w and 2 w + 1 (k-step w)");
    using TM = DmaTile<D, RB, 4>;
    __shared__ __align__(1024) char smem[2 * 2 * PLANE];
    __shared__ __align__(16) uint4 xch[2][KS][2][64];   // [buffer][k-step][hi, lo][lane]: B fragments of Sigma
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15,
              g4 = l >> 4;
    __builtin_assume(w >= 0 && w < 4);
    // workgroups go to the XCDs round robin: with BH a multiple of 8, the
    // column blocks of one (b, h) share an XCD (and its L2 copy of M)
    const int bh = blockIdx.x % a.BH, cbk = blockIdx.x / a.BH;
    const int col = BS * cbk + r16;
    const int nsteps = a.nseg - 1;
    uint32_t oM[TM::COUNT];
    TM::offsets(oM, RB, w, l);
    auto dma_m = [&](int s, char* buf) __attribute__((always_inline)) {
        const char* src = reinterpret_cast<const char*>(a.segM + ((size_t)bh * a.nseg + s) * 2 * D * D);
        TM::issue_s(src, oM, buf, w);
        TM::issue_s(src + PLANE, oM, buf + PLANE, w);
    };
    // the segment whose map step q applies, and where its result goes
    auto seg_of = [&](int q) __attribute__((always_inline)) { return REV ? a.nseg - 1 - q : q; };
    auto out_of = [&](int q) __attribute__((always_inline)) { return REV ? a.nseg - 2 - q : q + 1; };
    // rows BS i + 4 g4 .. + 3, i = 2 w + u, of the lane's column
    auto load_x = [&](int s, f32x4 (&X)[2]) __attribute__((always_inline)) {
        const float* xp = a.segX + ((size_t)bh * a.nseg + s) * D * D + (size_t)col * D;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float4 x = *reinterpret_cast<const float4*>(xp + BS * (2 * w + u) + 4 * g4);
            X[u] = f32x4{x.x, x.y, x.z, x.w};
        }
    };
    auto store_s = [&](int s, const f32x4 (&S)[2]) __attribute__((always_inline)) {
        float* out = a.segS + ((size_t)bh * a.nseg + s) * D * D + (size_t)col * D;
#pragma unroll
        for (int u = 0; u < 2; ++u)
            *reinterpret_cast<float4*>(out + BS * (2 * w + u) + 4 * g4) = make_float4(S[u][0], S[u][1], S[u][2], S[u][3]);
    };
    // the wave's two tiles as the split B fragment of k-step w
    auto put_b = [&](int buf, const f32x4 (&S)[2]) __attribute__((always_inline)) {
        const Frag8 f = accfrag<3>(S[0], S[1]);
        xch[buf][w][0][l] = __builtin_bit_cast(uint4, f.h);
        xch[buf][w][1][l] = __builtin_bit_cast(uint4, f.l);
    };
    f32x4 S[2], Xn[2];
    const float* sin = REV ? a.dsf : a.s0;   // [BH][dv][dk]
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        S[u] = zero4();
        if (sin) {
            const float4 x =
                *reinterpret_cast<const float4*>(sin + ((size_t)bh * D + col) * D + BS * (2 * w + u) + 4 * g4);
            S[u] = f32x4{x.x, x.y, x.z, x.w};
        }
    }
    put_b(0, S);
    dma_m(seg_of(0), smem);
    load_x(seg_of(0), Xn);
    for (int s = 0; s < nsteps; ++s) {
        dma_wait<0>();
        lds_barrier();   // M of step s landed for every wave, the exchange buffer s & 1 written; the other M buffer is free
        if (s > 0) store_s(out_of(s - 1), S);   // the previous step's result
        if (s + 1 < nsteps) dma_m(seg_of(s + 1), smem + ((s + 1) & 1) * 2 * PLANE);
        f32x4 Xc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) Xc[u] = Xn[u];
        if (s + 1 < nsteps) load_x(seg_of(s + 1), Xn);
        const ST* Mh = reinterpret_cast<const ST*>(smem + (s & 1) * 2 * PLANE);
        const ST* Ml = reinterpret_cast<const ST*>(smem + (s & 1) * 2 * PLANE + PLANE);
        Frag8 B[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            B[k].h = __builtin_bit_cast(bf16x8, xch[s & 1][k][0][l]);
            B[k].l = __builtin_bit_cast(bf16x8, xch[s & 1][k][1][l]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = 2 * w + u;
            f32x4 acc = Xc[u];
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                Frag8 A;
                if constexpr (REV) {
                    A.h = ldfrag_sw<RB>(Mh, BS * i, 32 * k).h;    // A[i][k] = M^T[i][k]
                    A.l = ldfrag_sw<RB>(Ml, BS * i, 32 * k).h;
                } else {
                    A.h = ldfragT_sw<RB>(Mh, BS * i, 32 * k).h;   // A[dk_out][dk_in] = M^T[dk_in][dk_out]
                    A.l = ldfragT_sw<RB>(Ml, BS * i, 32 * k).h;
                }
                acc = mma<3>(A, B[k], acc);
            }
            S[u] = acc;
        }
        // buffer (s + 1) & 1 was last read in step s - 1, before this step's barrier
        put_b((s + 1) & 1, S);
    }
    if (nsteps > 0) store_s(out_of(nsteps - 1), S);
}

// waves per workgroup of the segment maps and the segment forwards (eight: two
// per SIMD; four waves of 32 columns each read half the LDS operand bytes per
// step but measured slower, 186 against 155 us for config 3's pass C)
constexpr int SEG_NW = 8;

void seg_plan(int BH, int nc, int* nseg, int* seg_len) {
    // Fill about SEG_TARGET_WG workgroups (the MI355X's CU count: a fixed design
    // constant, so that the plan -- and with it the workspace size and the
    // result -- depends on the shape only), with at least SEG_MIN_LEN chunks
    // per segment.
    constexpr int SEG_TARGET_WG = 256, SEG_MIN_LEN = 4;
    int ns = BH > 0 ? SEG_TARGET_WG / BH : 1;
    if (ns > nc / SEG_MIN_LEN) ns = nc / SEG_MIN_LEN;
    if (ns < 1) ns = 1;
    const int len = (nc + ns - 1) / ns;
    *seg_len = len;
    *nseg = (nc + len - 1) / len;
}

hipError_t launch_seg_map(const SegArgs& a, hipStream_t st) {
    if (a.nseg < 2) return hipSuccess;
    hipLaunchKernelGGL((kda_segchain_kernel<128, 1, SEG_NW>), dim3(a.BH * (a.all_maps ? a.nseg : a.nseg - 1)),
                       dim3(64 * SEG_NW), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_seg_scan(const SegArgs& a, hipStream_t st) {
    if (a.nseg < 2) return hipSuccess;
    hipLaunchKernelGGL((kda_segscan_kernel<128>), dim3(a.BH * (128 / BS)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_seg_rscan(const SegArgs& a, hipStream_t st) {
    if (a.nseg < 2) return hipSuccess;
    hipLaunchKernelGGL((kda_segscan_kernel<128, true>), dim3(a.BH * (128 / BS)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_seg_states(const SegArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((kda_segchain_kernel<128, 2, SEG_NW>), dim3(a.BH * a.nseg), dim3(64 * SEG_NW), 0, st,
                       a);
    return hipGetLastError();
}

hipError_t launch_seg_fwd(const SegArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((kda_segchain_kernel<128, 0, SEG_NW>), dim3(a.BH * a.nseg), dim3(64 * SEG_NW), 0, st,
                       a);
    return hipGetLastError();
}

}  // namespace kda
