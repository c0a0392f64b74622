// kda_recur.hip -- the two sequential (inter-chunk) recurrences of the KDA op.
//
// One 256-thread workgroup per (batch, head) walks the chunks in order; wave w
// owns dv tiles w, w+4, ... of the state, which stays in accumulator VGPRs as
// fp32 for the whole sequence.  The chunk's shared operands (workspace slabs
// written by the prep kernel) are staged in LDS with 16-byte coalesced loads;
// the next chunk's slabs are loaded into registers while the current chunk is
// computed and land in the other half of a double buffer (single buffer plus a
// second barrier when two do not fit in 160 KB).  Per-chunk outputs go through
// an LDS staging tile and leave as coalesced 16-byte stores.
//
//   kda_recur_kernel  (state orientation S[dk][dv])
//       V' = U - W S;  O = Qp S + Aqk V';  S <- diag(e^G) S + Kb^T V'
//     MODE 0 writes O and the final state -- the chunk loop of
//     nope_gdn_mlx.py:2408-2451 (fused solve/finalize 1519-1942) with the
//     triangular solve hoisted into the prep kernel.
//     MODE 1 writes the chunk-start states h and V' for the backward instead.
//   kda_dh_kernel  (reverse order)
//       dV' = Aqk^T dO + Kb dS;  dS <- diag(e^G) dS + Qp^T dO - W^T dV'
//     writing dS at each chunk end and dV'; the final dS is dS0 -- the state
//     carry of nope_gdn_mlx.py:2705-2706 in W/U form.
#include "kda_internal.h"

namespace kda {

// Compiler-only fence: keeps the LDS writes of the prefetched chunk after the
// current chunk's compute.  Without it the writes are hoisted next to their
// loads, which turns the prefetch into a full memory-latency stall.
__device__ __forceinline__ void order_after_compute() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ Frag8 negfrag(Frag8 f) {
    uint4 u = __builtin_bit_cast(uint4, f.h);
    u.x ^= 0x80008000u; u.y ^= 0x80008000u; u.z ^= 0x80008000u; u.w ^= 0x80008000u;
    f.h = __builtin_bit_cast(bf16x8, u);
    uint4 v = __builtin_bit_cast(uint4, f.l);
    v.x ^= 0x80008000u; v.y ^= 0x80008000u; v.z ^= 0x80008000u; v.w ^= 0x80008000u;
    f.l = __builtin_bit_cast(bf16x8, v);
    return f;
}

// LDS geometry of one buffer (operand set + output staging)
// LDS geometry: NBUF operand sets (one chunk's slabs each) followed by NBUF
// output staging tiles.  Rows are padded by 16 bytes against bank conflicts.
// A workgroup owns DC = D / CS state columns; U and the outputs are DC wide.
template <int D, typename ST, int MODE, int CS>
struct RecurLayout {
    static constexpr int DC = D / CS;
    static constexpr int PS = 16 / (int)sizeof(ST);
    static constexpr int LDR = D + PS;               // rows of [C][D] / [D][D] tiles
    static constexpr int LDU = DC + PS;              // rows of [C][DC] tiles (U, outputs)
    static constexpr int LDC = C + PS;               // rows of [D][C] / [C][C] tiles
    static constexpr int W_OFF = 0;
    static constexpr int U_OFF = W_OFF + C * LDR;
    static constexpr int QP_OFF = U_OFF + C * LDU;
    static constexpr int KBT_OFF = QP_OFF + (MODE == 0 ? C * LDR : 0);
    static constexpr int AQK_OFF = KBT_OFF + D * LDC;
    static constexpr int SET_ELEMS = AQK_OFF + (MODE == 0 ? C * LDC : 0);
    static constexpr int EG_BYTE = SET_ELEMS * (int)sizeof(ST);
    static constexpr int SET_BYTES = (EG_BYTE + D * 4 + 15) & ~15;
    static constexpr int STG_ELEMS = (MODE == 0) ? C * LDU : D * LDU + C * LDU;   // O | h, V'
    static constexpr int STG_BYTES = (STG_ELEMS * (int)sizeof(ST) + 15) & ~15;
    static constexpr int NBUF = (2 * SET_BYTES + 2 * STG_BYTES <= 160 * 1024) ? 2 : 1;
    static constexpr int STG_OFF = NBUF * SET_BYTES;
    static constexpr int BYTES = STG_OFF + NBUF * STG_BYTES;
};

template <int D, typename ST>
struct DhLayout {
    static constexpr int PS = 16 / (int)sizeof(ST);
    static constexpr int LDR = D + PS, LDC = C + PS;
    static constexpr int AQKT_OFF = 0;
    static constexpr int KB_OFF = AQKT_OFF + C * LDC;
    static constexpr int QPT_OFF = KB_OFF + C * LDR;
    static constexpr int WT_OFF = QPT_OFF + D * LDC;
    static constexpr int DO_OFF = WT_OFF + D * LDC;
    static constexpr int SET_ELEMS = DO_OFF + C * LDR;
    static constexpr int EG_BYTE = SET_ELEMS * (int)sizeof(ST);
    static constexpr int SET_BYTES = (EG_BYTE + D * 4 + 15) & ~15;
    static constexpr int STG_ELEMS = D * LDR + C * LDR;      // dh, dV'
    static constexpr int STG_BYTES = (STG_ELEMS * (int)sizeof(ST) + 15) & ~15;
    static constexpr int NBUF = (2 * SET_BYTES + 2 * STG_BYTES <= 160 * 1024) ? 2 : 1;
    static constexpr int STG_OFF = NBUF * SET_BYTES;
    static constexpr int BYTES = STG_OFF + NBUF * STG_BYTES;
};

// ----------------------------------------------------------------------------
// forward recurrence / chunk-start state recompute
//
// Loop of chunk n (NBUF = 2):
//   issue the 16-byte loads of chunk n+1's slabs into registers;
//   issue the coalesced stores of chunk n-1's staged outputs (after the loads,
//   so waiting for the loads never waits for the stores);
//   compute chunk n from LDS set n&1 into staging tile n&1;
//   wait for the loads, write them to LDS set (n+1)&1; barrier.
// With NBUF = 1 an extra barrier separates the compute from the overwrite.
// ----------------------------------------------------------------------------
template <int D, typename ST, int PREC, int MODE, int CS>
__global__ __launch_bounds__(256) void kda_recur_kernel(const RecurArgs a) {
    using Lay = RecurLayout<D, ST, MODE, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, TPW = (NTW + 3) / 4;
    constexpr int LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC;
    __shared__ __align__(16) unsigned char smem[Lay::BYTES];

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    const int bh = blockIdx.x / CS, c0 = (blockIdx.x - bh * CS) * DC;
    const int b = bh / a.H, h = bh - b * a.H;
    const ST* gW = static_cast<const ST*>(a.W);
    const ST* gU = static_cast<const ST*>(a.U);
    const ST* gQp = static_cast<const ST*>(a.Qp);
    const ST* gKbT = static_cast<const ST*>(a.KbT);
    const ST* gAqk = static_cast<const ST*>(a.Aqk);

    auto set = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + buf * Lay::SET_BYTES); };
    auto seg = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<float*>(smem + buf * Lay::SET_BYTES + Lay::EG_BYTE); };
    auto stg = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + Lay::STG_OFF + sb * Lay::STG_BYTES); };

    // wave w owns local state columns lc = 16 (w + 4 j) + r16, global column c0 + lc
    bool has[TPW];
    int lcol[TPW], col[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        has[j] = (NTW % 4 == 0) || (w + 4 * j) < NTW;
        lcol[j] = (w + 4 * j) * BS + r16;
        col[j] = c0 + lcol[j];
    }

    // fp32 state tiles: rows d = 16 mt + 4 g4 + e, column col[j]
    f32x4 S[TPW][NT];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            S[j][mt] = zero4();
            if (has[j] && a.s0) {
                const float4 x =
                    *reinterpret_cast<const float4*>(a.s0 + ((size_t)bh * D + col[j]) * D + BS * mt + 4 * g4);
                S[j][mt] = f32x4{x.x, x.y, x.z, x.w};
            }
        }

    Tile<ST, C, D> pW, pQp;
    Tile<ST, C, DC> pU;
    Tile<ST, D, C> pKbT;
    Tile<ST, C, C> pAqk;
    Tile<float, 1, D> pEg;

    auto issue = [&](int n) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * a.nc + n;
        pW.load(gW + ch * C * D, D);
        pU.load(gU + ch * C * D + c0, D);
        pKbT.load(gKbT + ch * C * D, C);
        pEg.load(a.eG + ch * D, D);
        if constexpr (MODE == 0) {
            pQp.load(gQp + ch * C * D, D);
            pAqk.load(gAqk + ch * C * C, C);
        }
    };
    auto commit = [&](int buf) __attribute__((always_inline)) {
        pW.store(set(buf) + Lay::W_OFF, LDR);
        pU.store(set(buf) + Lay::U_OFF, LDU);
        pKbT.store(set(buf) + Lay::KBT_OFF, LDC);
        pEg.store(seg(buf), D);
        if constexpr (MODE == 0) {
            pQp.store(set(buf) + Lay::QP_OFF, LDR);
            pAqk.store(set(buf) + Lay::AQK_OFF, LDC);
        }
    };
    auto flush = [&](int n) __attribute__((always_inline)) {   // stores of chunk n's staged outputs
        const ST* sst = stg((Lay::NBUF == 2) ? (n & 1) : 0);
        if constexpr (MODE == 0) {
            const int t0 = n * C, valid = min(C, a.T - t0);
            tile_out<ST, C, DC>(sst, LDU, static_cast<ST*>(a.o) + (((size_t)b * a.T + t0) * a.H + h) * D + c0,
                                (size_t)a.H * D, valid);
        } else {
            const size_t ch = (size_t)bh * a.nc + n;
            tile_out<ST, D, DC>(sst, LDU, static_cast<ST*>(a.h) + ch * D * D + c0, D, D);
            tile_out<ST, C, DC>(sst + D * LDU, LDU, static_cast<ST*>(a.Vp) + ch * C * D + c0, D, C);
        }
    };

    issue(0);
    commit(0);
    __syncthreads();

    for (int n = 0; n < a.nc; ++n) {
        const int buf = (Lay::NBUF == 2) ? (n & 1) : 0;
        // RPHASE 0
        if (n + 1 < a.nc) issue(n + 1);
        if (Lay::NBUF == 2 && n > 0) flush(n - 1);

        const ST* sW = set(buf) + Lay::W_OFF;
        const ST* sU = set(buf) + Lay::U_OFF;
        const ST* sKbT = set(buf) + Lay::KBT_OFF;
        const float* seG = seg(buf);
        ST* sst = stg(buf);

        // All A fragments of this chunk are read from LDS first (one wait),
        // then the MFMA chain runs without LDS round trips in between.
        Frag8 Aw[NB][D / 32], Akb[NT][C / 32], Aq[NB][D / 32], Aa[NB][C / 32];
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Aw[m][ks] = ldfrag<PREC, ST>(sW, LDR, BS * m, 32 * ks);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Akb[mt][ks] = ldfrag<PREC, ST>(sKbT, LDC, BS * mt, 32 * ks);
        if constexpr (MODE == 0) {
            const ST* sQp = set(buf) + Lay::QP_OFF;
            const ST* sAqk = set(buf) + Lay::AQK_OFF;
#pragma unroll
            for (int m = 0; m < NB; ++m) {
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) Aq[m][ks] = ldfrag<PREC, ST>(sQp, LDR, BS * m, 32 * ks);
#pragma unroll
                for (int ks = 0; ks <= m / 2; ++ks) Aa[m][ks] = ldfrag<PREC, ST>(sAqk, LDC, BS * m, 32 * ks);
            }
        }
        f32x4 Vp[TPW][NB];
        Frag8 Bs[TPW][D / 32], Bn[TPW][D / 32];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) Vp[j][m][e] = ld1<ST>(sU + (BS * m + 4 * g4 + e) * LDU + lcol[j]);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                Bs[j][ks] = accfrag<PREC>(S[j][2 * ks], S[j][2 * ks + 1]);
                Bn[j][ks] = accfrag<PREC>(negacc(S[j][2 * ks]), negacc(S[j][2 * ks + 1]));
            }
        }
        __builtin_amdgcn_sched_barrier(0);

        // V' = U - W S
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
#pragma unroll
                for (int j = 0; j < TPW; ++j)
                    if (has[j]) Vp[j][m] = mma<PREC>(Aw[m][ks], Bn[j][ks], Vp[j][m]);
        Frag8 Bv[TPW][C / 32];
#pragma unroll
        for (int j = 0; j < TPW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bv[j][ks] = accfrag<PREC>(Vp[j][2 * ks], Vp[j][2 * ks + 1]);

        // S <- diag(e^G) S + Kb^T V'  (issued before O: it is on the critical path)
        f32x4 Snew[TPW][NT];
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            const float4 eg = *reinterpret_cast<const float4*>(seG + BS * mt + 4 * g4);
#pragma unroll
            for (int j = 0; j < TPW; ++j) {
                Snew[j][mt] = f32x4{S[j][mt][0] * eg.x, S[j][mt][1] * eg.y, S[j][mt][2] * eg.z, S[j][mt][3] * eg.w};
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks)
                    if (has[j]) Snew[j][mt] = mma<PREC>(Akb[mt][ks], Bv[j][ks], Snew[j][mt]);
            }
        }

        if constexpr (MODE == 0) {
            // O = Qp S + Aqk V'
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                f32x4 O[TPW];
#pragma unroll
                for (int j = 0; j < TPW; ++j) {
                    O[j] = zero4();
                    if (has[j]) {
#pragma unroll
                        for (int ks = 0; ks < D / 32; ++ks) O[j] = mma<PREC>(Aq[m][ks], Bs[j][ks], O[j]);
#pragma unroll
                        for (int ks = 0; ks <= m / 2; ++ks) O[j] = mma<PREC>(Aa[m][ks], Bv[j][ks], O[j]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) st1<ST>(sst + (BS * m + 4 * g4 + e) * LDU + lcol[j], O[j][e]);
                    }
                }
            }
        } else {
            ST* hst = sst;
            ST* vst = sst + D * LDU;
#pragma unroll
            for (int j = 0; j < TPW; ++j)
                if (has[j]) {
#pragma unroll
                    for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) st1<ST>(hst + (BS * mt + 4 * g4 + e) * LDU + lcol[j], S[j][mt][e]);
#pragma unroll
                    for (int m = 0; m < NB; ++m)
#pragma unroll
                        for (int e = 0; e < 4; ++e) st1<ST>(vst + (BS * m + 4 * g4 + e) * LDU + lcol[j], Vp[j][m][e]);
                }
        }
#pragma unroll
        for (int j = 0; j < TPW; ++j)
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) S[j][mt] = Snew[j][mt];

        order_after_compute();
        // RPHASE 1
        if constexpr (Lay::NBUF == 2) {
            if (n + 1 < a.nc) commit(buf ^ 1);
            // RPHASE 2
            __syncthreads();
            // RPHASE 3
        } else {
            __syncthreads();
            flush(n);
            if (n + 1 < a.nc) commit(0);
            __syncthreads();
        }
    }
    if (Lay::NBUF == 2) flush(a.nc - 1);

    if (MODE == 0 && a.s_final) {
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (has[j])
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
                    *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + col[j]) * D + BS * mt + 4 * g4) =
                        make_float4(S[j][mt][0], S[j][mt][1], S[j][mt][2], S[j][mt][3]);
    }
}

// ----------------------------------------------------------------------------
// reverse state recurrence (same pipeline, chunks in reverse order)
// ----------------------------------------------------------------------------
template <int D, typename ST, int PREC>
__global__ __launch_bounds__(256) void kda_dh_kernel(const DhArgs a) {
    using Lay = DhLayout<D, ST>;
    constexpr int NT = D / BS, TPW = (NT + 3) / 4, LDR = Lay::LDR, LDC = Lay::LDC;
    __shared__ __align__(16) unsigned char smem[Lay::BYTES];

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    const int bh = blockIdx.x, b = bh / a.H, h = bh - b * a.H;
    const ST* gAqkT = static_cast<const ST*>(a.AqkT);
    const ST* gKb = static_cast<const ST*>(a.Kb);
    const ST* gQpT = static_cast<const ST*>(a.QpT);
    const ST* gWT = static_cast<const ST*>(a.WT);
    const ST* gdO = static_cast<const ST*>(a.dout);

    auto set = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + buf * Lay::SET_BYTES); };
    auto seg = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<float*>(smem + buf * Lay::SET_BYTES + Lay::EG_BYTE); };
    auto stg = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + Lay::STG_OFF + sb * Lay::STG_BYTES); };

    bool has[TPW];
    int col[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        has[j] = (NT % 4 == 0) || (w + 4 * j) < NT;
        col[j] = (w + 4 * j) * BS + r16;
    }

    f32x4 dS[TPW][NT];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            dS[j][mt] = zero4();
            if (has[j] && a.dsf) {
                const float4 x =
                    *reinterpret_cast<const float4*>(a.dsf + ((size_t)bh * D + col[j]) * D + BS * mt + 4 * g4);
                dS[j][mt] = f32x4{x.x, x.y, x.z, x.w};
            }
        }

    Tile<ST, C, C> pAqkT;
    Tile<ST, C, D> pKb, pdO;
    Tile<ST, D, C> pQpT, pWT;
    Tile<float, 1, D> pEg;

    auto issue = [&](int n) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * a.nc + n;
        const int t0 = n * C, valid = min(C, a.T - t0);
        pAqkT.load(gAqkT + ch * C * C, C);
        pKb.load(gKb + ch * C * D, D);
        pQpT.load(gQpT + ch * C * D, C);
        pWT.load(gWT + ch * C * D, C);
        pEg.load(a.eG + ch * D, D);
        pdO.load(gdO + (((size_t)b * a.T + t0) * a.H + h) * D, (size_t)a.H * D, valid);
    };
    auto commit = [&](int buf) __attribute__((always_inline)) {
        pAqkT.store(set(buf) + Lay::AQKT_OFF, LDC);
        pKb.store(set(buf) + Lay::KB_OFF, LDR);
        pQpT.store(set(buf) + Lay::QPT_OFF, LDC);
        pWT.store(set(buf) + Lay::WT_OFF, LDC);
        pdO.store(set(buf) + Lay::DO_OFF, LDR);
        pEg.store(seg(buf), D);
    };
    auto flush = [&](int it, int n) __attribute__((always_inline)) {   // stores of chunk n (loop step it)
        const ST* sst = stg((Lay::NBUF == 2) ? (it & 1) : 0);
        const size_t ch = (size_t)bh * a.nc + n;
        tile_out<ST, D, D>(sst, LDR, static_cast<ST*>(a.dh) + ch * D * D, D, D);
        tile_out<ST, C, D>(sst + D * LDR, LDR, static_cast<ST*>(a.dVp) + ch * C * D, D, C);
    };

    issue(a.nc - 1);
    commit(0);
    __syncthreads();

    for (int it = 0; it < a.nc; ++it) {
        const int n = a.nc - 1 - it;
        const int buf = (Lay::NBUF == 2) ? (it & 1) : 0;
        if (n > 0) issue(n - 1);
        if (Lay::NBUF == 2 && it > 0) flush(it - 1, n + 1);

        const ST* sAqkT = set(buf) + Lay::AQKT_OFF;
        const ST* sKb = set(buf) + Lay::KB_OFF;
        const ST* sQpT = set(buf) + Lay::QPT_OFF;
        const ST* sWT = set(buf) + Lay::WT_OFF;
        const ST* sdO = set(buf) + Lay::DO_OFF;
        const float* seG = seg(buf);
        ST* dhst = stg(buf);
        ST* dvst = dhst + D * LDR;

        Frag8 Aat[NB][C / 32], Akb[NB][D / 32], Aqt[NT][C / 32], Awt[NT][C / 32];
#pragma unroll
        for (int m = 0; m < NB; ++m) {
#pragma unroll
            for (int ks = m / 2; ks < C / 32; ++ks) Aat[m][ks] = ldfrag<PREC, ST>(sAqkT, LDC, BS * m, 32 * ks);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Akb[m][ks] = ldfrag<PREC, ST>(sKb, LDR, BS * m, 32 * ks);
        }
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) {
                Aqt[mt][ks] = ldfrag<PREC, ST>(sQpT, LDC, BS * mt, 32 * ks);
                Awt[mt][ks] = ldfrag<PREC, ST>(sWT, LDC, BS * mt, 32 * ks);
            }
        Frag8 Bo[TPW][C / 32], Bs[TPW][D / 32];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            f32x4 dO[NB];
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) dO[m][e] = ld1<ST>(sdO + (BS * m + 4 * g4 + e) * LDR + col[j]);
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bo[j][ks] = accfrag<PREC>(dO[2 * ks], dO[2 * ks + 1]);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = accfrag<PREC>(dS[j][2 * ks], dS[j][2 * ks + 1]);
            if (has[j])
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) st1<ST>(dhst + (BS * mt + 4 * g4 + e) * LDR + col[j], dS[j][mt][e]);
        }
        __builtin_amdgcn_sched_barrier(0);

        // dV' = Aqk^T dO + Kb dS
        f32x4 dV[TPW][NB];
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int j = 0; j < TPW; ++j) {
                dV[j][m] = zero4();
                if (has[j]) {
#pragma unroll
                    for (int ks = m / 2; ks < C / 32; ++ks) dV[j][m] = mma<PREC>(Aat[m][ks], Bo[j][ks], dV[j][m]);
#pragma unroll
                    for (int ks = 0; ks < D / 32; ++ks) dV[j][m] = mma<PREC>(Akb[m][ks], Bs[j][ks], dV[j][m]);
                }
            }
        // dS <- diag(e^G) dS + Qp^T dO - W^T dV'
        Frag8 Bvn[TPW][C / 32];
#pragma unroll
        for (int j = 0; j < TPW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks)
                Bvn[j][ks] = accfrag<PREC>(negacc(dV[j][2 * ks]), negacc(dV[j][2 * ks + 1]));
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            const float4 eg = *reinterpret_cast<const float4*>(seG + BS * mt + 4 * g4);
#pragma unroll
            for (int j = 0; j < TPW; ++j) {
                dS[j][mt][0] *= eg.x; dS[j][mt][1] *= eg.y; dS[j][mt][2] *= eg.z; dS[j][mt][3] *= eg.w;
                if (has[j]) {
#pragma unroll
                    for (int ks = 0; ks < C / 32; ++ks) {
                        dS[j][mt] = mma<PREC>(Aqt[mt][ks], Bo[j][ks], dS[j][mt]);
                        dS[j][mt] = mma<PREC>(Awt[mt][ks], Bvn[j][ks], dS[j][mt]);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (has[j])
#pragma unroll
                for (int m = 0; m < NB; ++m)
#pragma unroll
                    for (int e = 0; e < 4; ++e) st1<ST>(dvst + (BS * m + 4 * g4 + e) * LDR + col[j], dV[j][m][e]);

        order_after_compute();
        if constexpr (Lay::NBUF == 2) {
            if (n > 0) commit(buf ^ 1);
            __syncthreads();
        } else {
            __syncthreads();
            flush(it, n);
            if (n > 0) commit(0);
            __syncthreads();
        }
    }
    if (Lay::NBUF == 2) flush(a.nc - 1, 0);

    if (a.ds0) {
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (has[j])
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
                    *reinterpret_cast<float4*>(a.ds0 + ((size_t)bh * D + col[j]) * D + BS * mt + 4 * g4) =
                        make_float4(dS[j][mt][0], dS[j][mt][1], dS[j][mt][2], dS[j][mt][3]);
    }
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
// D = 128 splits the state's dv columns over two workgroups per (batch, head)
template <int D, typename ST, int MODE>
static hipError_t launch_recur_t(const RecurArgs& a, hipStream_t st) {
    constexpr int PREC = std::is_same<ST, float>::value ? 3 : 1;
    constexpr int CS = (D >= 128) ? 2 : 1;
    hipLaunchKernelGGL((kda_recur_kernel<D, ST, PREC, MODE, CS>), dim3(a.BH * CS), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int D, typename ST>
static hipError_t launch_dh_t(const DhArgs& a, hipStream_t st) {
    constexpr int PREC = std::is_same<ST, float>::value ? 3 : 1;
    hipLaunchKernelGGL((kda_dh_kernel<D, ST, PREC>), dim3(a.BH), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_recur(const RecurArgs& a, int D, int in_bf16, int mode, hipStream_t st) {
#define KDA_RECUR_CASE(DD)                                                                        \
    if (D == DD) {                                                                                \
        if (mode == 0) return in_bf16 ? launch_recur_t<DD, uint16_t, 0>(a, st)                    \
                                      : launch_recur_t<DD, float, 0>(a, st);                      \
        return in_bf16 ? launch_recur_t<DD, uint16_t, 1>(a, st) : launch_recur_t<DD, float, 1>(a, st); \
    }
    KDA_RECUR_CASE(32)
    KDA_RECUR_CASE(64)
#undef KDA_RECUR_CASE
    // the backward (MODE 1) supports D <= 64
    if (D == 128 && mode == 0)
        return in_bf16 ? launch_recur_t<128, uint16_t, 0>(a, st) : launch_recur_t<128, float, 0>(a, st);
    return hipErrorInvalidValue;
}

hipError_t launch_dh(const DhArgs& a, int D, int in_bf16, hipStream_t st) {
    if (D == 32) return in_bf16 ? launch_dh_t<32, uint16_t>(a, st) : launch_dh_t<32, float>(a, st);
    if (D == 64) return in_bf16 ? launch_dh_t<64, uint16_t>(a, st) : launch_dh_t<64, float>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace kda
