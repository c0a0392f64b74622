// kda_recur.hip -- the sequential (inter-chunk) recurrences of the KDA op.
//
// Each walks the chunks of one (batch, head) in order, with the state in fp32
// MFMA accumulators for the whole sequence and the chunk's workspace slabs
// (written by the prep kernel) staged in LDS.  The state orientation inside the
// kernels is Sigma = S^T, [dk][dv].
//
//   forward (MODE 0) and chunk-start state recompute (MODE 1)
//       V' = U - W Sigma;  O = Qp Sigma + Aqk V';  Sigma <- diag(e^G) Sigma + Kb^T V'
//     MODE 0 writes O and the final state -- the chunk loop of
//     nope_gdn_mlx.py:2408-2451 (fused solve/finalize 1519-1942) with the
//     triangular solve hoisted into the prep kernel; MODE 1 writes the
//     chunk-start states h for the backward.
//   reverse state carry
//       dV' = Aqk^T dO + Kb dSigma;  dSigma <- diag(e^G) dSigma + Qp^T dO - W^T dV'
//     writing dSigma at each chunk end and dV'; the last dSigma is dS0 -- the
//     state carry of nope_gdn_mlx.py:2705-2706 in W/U form.
//
// Kernels by shape:
//   kda_recur4_kernel / kda_dh4_kernel  bf16, D = 64: two 8-wave workgroups per
//       (batch, head), each owning half of the dv columns; wave roles (state
//       chain | work beside it), slabs by LDS DMA three chunks ahead
//   kda_recur5_kernel  bf16, D = 64, forward with the layer's gated RMSNorm
//       fused into the O store: one 16-wave workgroup per (batch, head)
//   kda_recur3_kernel  bf16, D = 128 forward: four 4-wave workgroups per
//       (batch, head), 32 dv columns each
//   kda_recur2_kernel / kda_dh2_kernel  bf16, D = 32
//   kda_recur_kernel / kda_dh_kernel    fp32 inputs (the first, generic design:
//       one 256-thread workgroup per (batch, head), register-staged double buffer)
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

// A workgroup owns DC = D / CS columns of dS (its dO, dh and dV' tiles are DC
// wide); the operand slabs Aqk^T, Kb, Qp^T and W^T are whole.
template <int D, typename ST, int CS = 1>
struct DhLayout {
    static constexpr int DC = D / CS;
    static constexpr int PS = 16 / (int)sizeof(ST);
    static constexpr int LDR = D + PS, LDC = C + PS, LDU = DC + PS;
    static constexpr int AQKT_OFF = 0;
    static constexpr int KB_OFF = AQKT_OFF + C * LDC;
    static constexpr int QPT_OFF = KB_OFF + C * LDR;
    static constexpr int WT_OFF = QPT_OFF + D * LDC;
    static constexpr int DO_OFF = WT_OFF + D * LDC;
    static constexpr int SET_ELEMS = DO_OFF + C * LDU;
    static constexpr int EG_BYTE = SET_ELEMS * (int)sizeof(ST);
    static constexpr int SET_BYTES = (EG_BYTE + D * 4 + 15) & ~15;
    static constexpr int STG_ELEMS = D * LDU + C * LDU;      // dh, dV'
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
// The kernel body (kda_recur_kernel, kda_states_dh_kernel): workgroup wgi of
// the launch's recurrence workgroups, Lay::BYTES of LDS at smem.
template <int D, typename ST, int PREC, int MODE, int CS, bool EPI = false>
__device__ __forceinline__ void recur_body(const RecurArgs& a, unsigned char* smem, const int wgi) {
    using Lay = RecurLayout<D, ST, MODE, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, TPW = (NTW + 3) / 4;
    constexpr int LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC;

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    const int bh = wgi / CS, c0 = (wgi - bh * CS) * DC;
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
            ST* go = static_cast<ST*>(a.o) + (((size_t)b * a.T + t0) * a.H + h) * D + c0;
            if constexpr (EPI) {
                // whole rows (CS = 1): the gated RMSNorm on the staged tile, z read here
                static_assert(CS == 1, "the fused epilogue needs whole output rows");
                const size_t rb = (size_t)b * a.T + t0;
                tile_out_gated<ST, C, D>((int)threadIdx.x, sst, LDU, go, (size_t)a.H * D,
                                         static_cast<ST*>(a.y) + rb * a.ld_y + (size_t)h * D, (size_t)a.ld_y,
                                         static_cast<const ST*>(a.z) + rb * a.ld_z + (size_t)h * D,
                                         (size_t)a.ld_z, a.nw, a.eps, valid);
            } else {
                tile_out<ST, C, DC>(sst, LDU, go, (size_t)a.H * D, valid);
            }
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
template <int D, typename ST, int PREC, int MODE, int CS, bool EPI = false>
__global__ __launch_bounds__(256) void kda_recur_kernel(const RecurArgs a) {
    __shared__ __align__(16) unsigned char smem[RecurLayout<D, ST, MODE, CS>::BYTES];
    recur_body<D, ST, PREC, MODE, CS, EPI>(a, smem, blockIdx.x);
}

// CS > 1: CS workgroups per (batch, head), DC = D / CS columns each; every A
// fragment is then used by one column tile of a wave, so fragments are read
// from LDS where they are used instead of being held for the whole chunk (at
// D = 128 in fp32 the whole set would take about 430 VGPRs).
// SEGM: the chunks of one segment of a.seg_len chunks per workgroup (the loop
// is linear in dSigma, so segments compose; the segment's map on dSigma is the
// transpose of the forward segment map M).  SEGM 1: segments 1 .. nseg - 1
// from dSigma = 0, writing only the segment's end value X_rev (to a.segX, the
// reference orientation [dv][dk]); SEGM 2: every segment from its incoming
// dSigma (ds_final for the last segment, a.segS, the reverse scan's result,
// for the others), writing dh and dV' and, for segment 0, dS0.
// The kernel body (kda_dh_kernel, kda_states_dh_kernel): workgroup wgi of the
// launch's reverse-carry workgroups, Lay::BYTES of LDS at smem.
template <int D, typename ST, int PREC, int CS = 1, int SEGM = 0>
__device__ __forceinline__ void dh_body(const DhArgs& a, unsigned char* smem, const int wgi) {
    using Lay = DhLayout<D, ST, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, TPW = (NTW + 3) / 4;
    constexpr int LDR = Lay::LDR, LDC = Lay::LDC, LDU = Lay::LDU;
    constexpr bool HOLD = CS == 1;   // A fragments held in registers for the chunk
    static_assert(Lay::BYTES <= 160 * 1024, "reverse recurrence LDS");

    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    // the workgroup's segment: chunks n0 .. n0 + L - 1 (the whole sequence without SEGM)
    int wg = wgi, sgi = 0, n0 = 0, L = a.nc;
    if constexpr (SEGM != 0) {
        const int nsegw = (SEGM == 1) ? a.nseg - 1 : a.nseg;
        const int si = wg % nsegw;
        wg /= nsegw;
        sgi = (SEGM == 1) ? si + 1 : si;
        n0 = sgi * a.seg_len;
        L = min(a.nc, n0 + a.seg_len) - n0;
    }
    const int bh = wg / CS, c0 = (wg - bh * CS) * DC, b = bh / a.H, h = bh - b * a.H;
    const ST* gAqkT = static_cast<const ST*>(a.AqkT);
    const ST* gKb = static_cast<const ST*>(a.Kb);
    const ST* gQpT = static_cast<const ST*>(a.QpT);
    const ST* gWT = static_cast<const ST*>(a.WT);
    const ST* gdO = static_cast<const ST*>(a.dout);

    auto set = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + buf * Lay::SET_BYTES); };
    auto seg = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<float*>(smem + buf * Lay::SET_BYTES + Lay::EG_BYTE); };
    auto stg = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + Lay::STG_OFF + sb * Lay::STG_BYTES); };

    // column tile w + 4 j of the workgroup's DC columns; col: within the slice
    bool has[TPW];
    int col[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        has[j] = (NTW % 4 == 0) || (w + 4 * j) < NTW;
        col[j] = (w + 4 * j) * BS + r16;
    }

    // the incoming dSigma ([dv][dk] like ds_final): ds_final, or for SEGM 2 the
    // reverse scan's value at a segment's end; zero for SEGM 1
    const float* dsin = a.dsf ? a.dsf + (size_t)bh * D * D : nullptr;
    if constexpr (SEGM == 1) dsin = nullptr;
    if constexpr (SEGM == 2)
        if (sgi < a.nseg - 1) dsin = a.segS + ((size_t)bh * a.nseg + sgi) * D * D;
    f32x4 dS[TPW][NT];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
            dS[j][mt] = zero4();
            if (has[j] && dsin) {
                const float4 x = *reinterpret_cast<const float4*>(dsin + (size_t)(c0 + col[j]) * D + BS * mt + 4 * g4);
                dS[j][mt] = f32x4{x.x, x.y, x.z, x.w};
            }
        }

    Tile<ST, C, C> pAqkT;
    Tile<ST, C, D> pKb;
    Tile<ST, C, DC> pdO;
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
        pdO.load(gdO + (((size_t)b * a.T + t0) * a.H + h) * D + c0, (size_t)a.H * D, valid);
    };
    auto commit = [&](int buf) __attribute__((always_inline)) {
        pAqkT.store(set(buf) + Lay::AQKT_OFF, LDC);
        pKb.store(set(buf) + Lay::KB_OFF, LDR);
        pQpT.store(set(buf) + Lay::QPT_OFF, LDC);
        pWT.store(set(buf) + Lay::WT_OFF, LDC);
        pdO.store(set(buf) + Lay::DO_OFF, LDU);
        pEg.store(seg(buf), D);
    };
    auto flush = [&](int it, int n) __attribute__((always_inline)) {   // stores of chunk n (loop step it)
        if constexpr (SEGM == 1) return;   // the segment map writes only its end value
        const ST* sst = stg((Lay::NBUF == 2) ? (it & 1) : 0);
        const size_t ch = (size_t)bh * a.nc + n;
        tile_out<ST, D, DC>(sst, LDU, static_cast<ST*>(a.dh) + ch * D * D + c0, D, D);
        tile_out<ST, C, DC>(sst + D * LDU, LDU, static_cast<ST*>(a.dVp) + ch * C * D + c0, D, C);
    };

    issue(n0 + L - 1);
    commit(0);
    __syncthreads();

    for (int it = 0; it < L; ++it) {
        const int n = n0 + L - 1 - it;
        const int buf = (Lay::NBUF == 2) ? (it & 1) : 0;
        if (n > n0) issue(n - 1);
        if (Lay::NBUF == 2 && it > 0) flush(it - 1, n + 1);

        const ST* sAqkT = set(buf) + Lay::AQKT_OFF;
        const ST* sKb = set(buf) + Lay::KB_OFF;
        const ST* sQpT = set(buf) + Lay::QPT_OFF;
        const ST* sWT = set(buf) + Lay::WT_OFF;
        const ST* sdO = set(buf) + Lay::DO_OFF;
        const float* seG = seg(buf);
        ST* dhst = stg(buf);
        ST* dvst = dhst + D * LDU;

        Frag8 Aat[HOLD ? NB : 1][C / 32], Akb[HOLD ? NB : 1][D / 32], Aqt[HOLD ? NT : 1][C / 32],
            Awt[HOLD ? NT : 1][C / 32];
        if constexpr (HOLD) {
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
        }
        auto fAat = [&](int m, int ks) __attribute__((always_inline)) {
            if constexpr (HOLD) return Aat[m][ks]; else return ldfrag<PREC, ST>(sAqkT, LDC, BS * m, 32 * ks);
        };
        auto fAkb = [&](int m, int ks) __attribute__((always_inline)) {
            if constexpr (HOLD) return Akb[m][ks]; else return ldfrag<PREC, ST>(sKb, LDR, BS * m, 32 * ks);
        };
        auto fAqt = [&](int mt, int ks) __attribute__((always_inline)) {
            if constexpr (HOLD) return Aqt[mt][ks]; else return ldfrag<PREC, ST>(sQpT, LDC, BS * mt, 32 * ks);
        };
        auto fAwt = [&](int mt, int ks) __attribute__((always_inline)) {
            if constexpr (HOLD) return Awt[mt][ks]; else return ldfrag<PREC, ST>(sWT, LDC, BS * mt, 32 * ks);
        };
        Frag8 Bo[TPW][C / 32], Bs[TPW][D / 32];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            f32x4 dO[NB];
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dO[m][e] = has[j] ? ld1<ST>(sdO + (BS * m + 4 * g4 + e) * LDU + col[j]) : 0.f;
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bo[j][ks] = accfrag<PREC>(dO[2 * ks], dO[2 * ks + 1]);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = accfrag<PREC>(dS[j][2 * ks], dS[j][2 * ks + 1]);
            if (has[j])
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) st1<ST>(dhst + (BS * mt + 4 * g4 + e) * LDU + col[j], dS[j][mt][e]);
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
                    for (int ks = m / 2; ks < C / 32; ++ks) dV[j][m] = mma<PREC>(fAat(m, ks), Bo[j][ks], dV[j][m]);
#pragma unroll
                    for (int ks = 0; ks < D / 32; ++ks) dV[j][m] = mma<PREC>(fAkb(m, ks), Bs[j][ks], dV[j][m]);
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
                        dS[j][mt] = mma<PREC>(fAqt(mt, ks), Bo[j][ks], dS[j][mt]);
                        dS[j][mt] = mma<PREC>(fAwt(mt, ks), Bvn[j][ks], dS[j][mt]);
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
                    for (int e = 0; e < 4; ++e) st1<ST>(dvst + (BS * m + 4 * g4 + e) * LDU + col[j], dV[j][m][e]);

        order_after_compute();
        if constexpr (Lay::NBUF == 2) {
            if (n > n0) commit(buf ^ 1);
            __syncthreads();
        } else {
            __syncthreads();
            flush(it, n);
            if (n > n0) commit(0);
            __syncthreads();
        }
    }
    if (Lay::NBUF == 2) flush(L - 1, n0);

    if constexpr (SEGM == 1) {
        float* xo = a.segX + ((size_t)bh * a.nseg + sgi) * D * D;
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (has[j])
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
                    *reinterpret_cast<float4*>(xo + (size_t)(c0 + col[j]) * D + BS * mt + 4 * g4) =
                        make_float4(dS[j][mt][0], dS[j][mt][1], dS[j][mt][2], dS[j][mt][3]);
        return;
    }
    if (a.ds0 && sgi == 0) {
#pragma unroll
        for (int j = 0; j < TPW; ++j)
            if (has[j])
#pragma unroll
                for (int mt = 0; mt < NT; ++mt)
                    *reinterpret_cast<float4*>(a.ds0 + ((size_t)bh * D + c0 + col[j]) * D + BS * mt + 4 * g4) =
                        make_float4(dS[j][mt][0], dS[j][mt][1], dS[j][mt][2], dS[j][mt][3]);
    }
}

template <int D, typename ST, int PREC, int CS = 1, int SEGM = 0>
__global__ __launch_bounds__(256) void kda_dh_kernel(const DhArgs a) {
    __shared__ __align__(16) unsigned char smem[DhLayout<D, ST, CS>::BYTES];
    dh_body<D, ST, PREC, CS, SEGM>(a, smem, blockIdx.x);
}

// The backward's state recompute and reverse carry at bf16 D = 128 in one
// launch.  They are independent (the reverse carry does not read the states)
// and one workgroup of either fills a CU's LDS, so workgroups 0 .. 2 BH - 1
// recompute the states (two per (b, h), as kda_recur_kernel) and the next 2 BH
// run the reverse carry (two per (b, h), as kda_dh_kernel), side by side on
// 4 BH CUs instead of one kernel after the other.
__global__ __launch_bounds__(256) void kda_states_dh_kernel(const RecurArgs ra, const DhArgs da) {
    constexpr int B1 = RecurLayout<128, uint16_t, 1, 2>::BYTES, B2 = DhLayout<128, uint16_t, 2>::BYTES;
    __shared__ __align__(16) unsigned char smem[B1 > B2 ? B1 : B2];
    const int n1 = 2 * ra.BH;
    if ((int)blockIdx.x < n1)
        recur_body<128, uint16_t, 1, 1, 2>(ra, smem, blockIdx.x);
    else
        dh_body<128, uint16_t, 1, 2, 0>(da, smem, (int)blockIdx.x - n1);
}

// ----------------------------------------------------------------------------
// bf16 recurrences, row split and warp-specialised.
//
// CS workgroups per (batch, head) each own DC = D / CS state columns (the
// state update, V' and O are all column-separable).  A workgroup has 8 waves:
//   compute waves 0-3: wave w owns row block w of the chunk's [C][DC] tiles
//     (V', O / dV') and state row blocks w, w + 4, ... .  Per chunk the state
//     and then V' pass between them through LDS as bf16 B operands, transposed
//     so every fragment is two 8-byte reads;
//   memory waves 4-7: stream the chunk slabs (registers two chunks ahead,
//     committed to the other half of a double-buffered LDS set one chunk
//     ahead) and flush the staged outputs with coalesced 16-byte stores.
// Both roles meet at two barriers per chunk:
//   compute: [A] fragments, V' = U - W S, write V'^T [B] S <- diag(e^G) S +
//            Kb^T V', write S^T for the next chunk, O = Qp S + Aqk V' -> staging
//   memory:  [A] flush chunk n-1 [B] commit chunk n+1, load chunk n+2
// ----------------------------------------------------------------------------
template <int D, int MODE, int CS>
struct Recur2Layout {
    static constexpr int DC = D / CS, PS = 8;
    static constexpr int LDR = D + PS, LDU = DC + PS, LDC = C + PS;
    static constexpr int W_OFF = 0;
    static constexpr int U_OFF = W_OFF + C * LDR;
    static constexpr int QP_OFF = U_OFF + C * LDU;
    static constexpr int KBT_OFF = QP_OFF + (MODE == 0 ? C * LDR : 0);
    static constexpr int AQK_OFF = KBT_OFF + D * LDC;
    static constexpr int SET_ELEMS = AQK_OFF + (MODE == 0 ? C * LDC : 0);
    static constexpr int EG_BYTE = SET_ELEMS * 2;
    static constexpr int SET_BYTES = (EG_BYTE + D * 4 + 15) & ~15;
    static constexpr int XS_OFF = 2 * SET_BYTES;                 // S^T  [DC][LDR]
    static constexpr int XV_OFF = XS_OFF + DC * LDR * 2;         // V'^T [DC][LDC]
    static constexpr int STG_OFF = XV_OFF + DC * LDC * 2;
    static constexpr int STG_ELEMS = (MODE == 0) ? C * LDU : D * LDU;   // O | h
    static constexpr int STG_BYTES = (STG_ELEMS * 2 + 15) & ~15;
    static constexpr int NSTG = (MODE == 0) ? 2 : 3;            // staging tiles, by chunk % NSTG
    static constexpr int BYTES = STG_OFF + NSTG * STG_BYTES;
    static_assert(BYTES <= 160 * 1024, "recurrence LDS");
};

// the lane's 4 consecutive rows of an accumulator as 4 bf16 (8 bytes)
__device__ __forceinline__ uint2 pack4bf(const f32x4& x) {
    return make_uint2(pack2bf(x[0], x[1]), pack2bf(x[2], x[3]));
}

// one chunk's slabs for the forward recurrence, in registers of a memory wave
template <int D, int MODE, int CS>
struct Recur2Slabs {
    static constexpr int DC = D / CS;
    Tile<uint16_t, C, D> W, Qp;
    Tile<uint16_t, C, DC> U;
    Tile<uint16_t, D, C> KbT;
    Tile<uint16_t, C, C> Aqk;
    Tile<float, 1, D> eG;
};

template <int D, int MODE, int CS>
__global__ __launch_bounds__(512) void kda_recur2_kernel(const RecurArgs a) {
    using ST = uint16_t;
    using Lay = Recur2Layout<D, MODE, CS>;
    using Slabs = Recur2Slabs<D, MODE, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, MT = (NT + 3) / 4;
    constexpr int LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC;
    __shared__ __align__(16) unsigned char smem[Lay::BYTES];

    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lb / CS, c0 = (lb - bh * CS) * DC;
    const int b = bh / a.H, h = bh - b * a.H;

    auto set = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + buf * Lay::SET_BYTES); };
    auto seg = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<float*>(smem + buf * Lay::SET_BYTES + Lay::EG_BYTE); };
    auto stg = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + Lay::STG_OFF + sb * Lay::STG_BYTES); };
    ST* xs = reinterpret_cast<ST*>(smem + Lay::XS_OFF);
    ST* xv = reinterpret_cast<ST*>(smem + Lay::XV_OFF);

    if (wv >= 4) {
        // ---------------- memory waves ----------------
        const int mt = tid - 256;
        auto issue = [&](int n, Slabs& p) __attribute__((always_inline)) {
            const size_t ch = (size_t)bh * a.nc + n;
            p.W.load_at(mt, static_cast<const ST*>(a.W) + ch * C * D, D);
            p.U.load_at(mt, static_cast<const ST*>(a.U) + ch * C * D + c0, D);
            p.KbT.load_at(mt, static_cast<const ST*>(a.KbT) + ch * C * D, C);
            p.eG.load_at(mt, a.eG + ch * D, D);
            if constexpr (MODE == 0) {
                p.Qp.load_at(mt, static_cast<const ST*>(a.Qp) + ch * C * D, D);
                p.Aqk.load_at(mt, static_cast<const ST*>(a.Aqk) + ch * C * C, C);
            }
        };
        auto commit = [&](int buf, const Slabs& p) __attribute__((always_inline)) {
            p.W.store_at(mt, set(buf) + Lay::W_OFF, LDR);
            p.U.store_at(mt, set(buf) + Lay::U_OFF, LDU);
            p.KbT.store_at(mt, set(buf) + Lay::KBT_OFF, LDC);
            p.eG.store_at(mt, seg(buf), D);
            if constexpr (MODE == 0) {
                p.Qp.store_at(mt, set(buf) + Lay::QP_OFF, LDR);
                p.Aqk.store_at(mt, set(buf) + Lay::AQK_OFF, LDC);
            }
        };
        auto flush = [&](int n) __attribute__((always_inline)) {
            const ST* sst = stg(n % Lay::NSTG);
            if constexpr (MODE == 0) {
                const int t0 = n * C, valid = min(C, a.T - t0);
                tile_out_at<ST, C, DC>(mt, sst, LDU,
                                       static_cast<ST*>(a.o) + (((size_t)b * a.T + t0) * a.H + h) * D + c0,
                                       (size_t)a.H * D, valid);
            } else {
                const size_t ch = (size_t)bh * a.nc + n;
                tile_out_at<ST, D, DC>(mt, sst, LDU, static_cast<ST*>(a.h) + ch * D * D + c0, D, D);
            }
        };
        // Chunk c's slabs live in register set c % NS from their load (NS
        // chunks ahead) to their commit into LDS set c & 1 (one chunk ahead);
        // NS = 2 at D = 128, whose slabs would not fit three times.  The loop is
        // unrolled NS times so that every step names its register set and the
        // compiler can wait for exactly the loads that step commits.
        //   between A(n) and B(n): commit chunk n+1
        //   between B(n) and A(n+1): flush chunk n-1, load chunk n+1+NS
        constexpr int NS = (D >= 128) ? 2 : 3;
        Slabs p0, p1, p2;
        issue(0, p0);
        if (a.nc > 1) issue(1, p1);
        if (NS == 3 && a.nc > 2) issue(2, p2);
        commit(0, p0);
        if (a.nc > NS) issue(NS, p0);
        __syncthreads();                                       // P: chunk 0 committed
        auto step = [&](int n, Slabs& p) __attribute__((always_inline)) {   // p holds chunk n+1
            __syncthreads();                                   // A(n)
            if (n + 1 < a.nc) commit((n + 1) & 1, p);
            __syncthreads();                                   // B(n): chunk n+1 committed
            if (n > 0) flush(n - 1);
            if (n + 1 + NS < a.nc) issue(n + 1 + NS, p);
        };
        for (int n = 0; n < a.nc; n += NS) {
            step(n, p1);
            if (n + 1 < a.nc) step(n + 1, NS == 3 ? p2 : p0);
            if (NS == 3 && n + 2 < a.nc) step(n + 2, p0);
        }
        __syncthreads();
        flush(a.nc - 1);
        return;
    }

    // ---------------- compute waves ----------------
    const int w = wv, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    // state tiles: rows d = 16 mt[i] + 4 g4 + e, local columns 16 j + r16
    int mt[MT];
    bool own[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        mt[i] = w + 4 * i;
        own[i] = mt[i] < NT;
    }
    f32x4 S[MT][NTW];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            S[i][j] = zero4();
            if (own[i] && a.s0) {
                const float4 x = *reinterpret_cast<const float4*>(
                    a.s0 + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4);
                S[i][j] = f32x4{x.x, x.y, x.z, x.w};
            }
        }
    // S^T for the B operands (and, for the backward, the chunk-start state)
    auto put_state = [&](ST* sst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    *reinterpret_cast<uint2*>(xs + (BS * j + r16) * LDR + BS * mt[i] + 4 * g4) = pack4bf(S[i][j]);
                    if constexpr (MODE == 1)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            st1<ST>(sst + (BS * mt[i] + 4 * g4 + e) * LDU + BS * j + r16, S[i][j][e]);
                }
    };
    put_state(stg(0));

    // A operands of one chunk, read from its LDS set ahead of time
    Frag8 Aw[D / 32], Aq[D / 32], Aa[2], Akb[MT][C / 32];
    f32x4 Uv[NTW];
    float4 eg[MT];
    auto preload = [&](int buf) __attribute__((always_inline)) {
        const ST* sW = set(buf) + Lay::W_OFF;
        const ST* sU = set(buf) + Lay::U_OFF;
        const ST* sKbT = set(buf) + Lay::KBT_OFF;
        const float* seG = seg(buf);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) Aw[ks] = ldfrag<1, ST>(sW, LDR, BS * w, 32 * ks);
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) Uv[j][e] = ld1<ST>(sU + (BS * w + 4 * g4 + e) * LDU + BS * j + r16);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) Akb[i][ks] = ldfrag<1, ST>(sKbT, LDC, BS * mt[i], 32 * ks);
                eg[i] = *reinterpret_cast<const float4*>(seG + BS * mt[i] + 4 * g4);
            }
        if constexpr (MODE == 0) {
            const ST* sQp = set(buf) + Lay::QP_OFF;
            const ST* sAqk = set(buf) + Lay::AQK_OFF;
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Aq[ks] = ldfrag<1, ST>(sQp, LDR, BS * w, 32 * ks);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (ks <= w / 2) Aa[ks] = ldfrag<1, ST>(sAqk, LDC, BS * w, 32 * ks);
        }
    };
    __syncthreads();                                           // P
    preload(0);

    for (int n = 0; n < a.nc; ++n) {
        const int buf = n & 1;
        ST* sst = stg(n % Lay::NSTG);
        __syncthreads();                                       // A(n)

        Frag8 Bs[NTW][D / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = ldfrag<1, ST>(xs, LDR, BS * j, 32 * ks);
        // V' = U - W S, row block w
        f32x4 Vp[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            f32x4 P = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) P = mma<1>(Aw[ks], Bs[j][ks], P);
#pragma unroll
            for (int e = 0; e < 4; ++e) Vp[j][e] = Uv[j][e] - P[e];
            *reinterpret_cast<uint2*>(xv + (BS * j + r16) * LDC + BS * w + 4 * g4) = pack4bf(Vp[j]);
        }
        __syncthreads();                                       // B(n)

        Frag8 Bv[NTW][C / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bv[j][ks] = ldfrag<1, ST>(xv, LDC, BS * j, 32 * ks);
        // S <- diag(e^G) S + Kb^T V'  (first: the next chunk waits for it)
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    S[i][j] = f32x4{S[i][j][0] * eg[i].x, S[i][j][1] * eg[i].y, S[i][j][2] * eg[i].z,
                                    S[i][j][3] * eg[i].w};
#pragma unroll
                    for (int ks = 0; ks < C / 32; ++ks) S[i][j] = mma<1>(Akb[i][ks], Bv[j][ks], S[i][j]);
                }
            }
        if (n + 1 < a.nc) put_state(stg((n + 1) % Lay::NSTG));
        if constexpr (MODE == 0) {
            // O = Qp S + Aqk V', row block w (the chunk-start state is in Bs)
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                f32x4 O = zero4();
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) O = mma<1>(Aq[ks], Bs[j][ks], O);
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    if (ks <= w / 2) O = mma<1>(Aa[ks], Bv[j][ks], O);
#pragma unroll
                for (int e = 0; e < 4; ++e) st1<ST>(sst + (BS * w + 4 * g4 + e) * LDU + BS * j + r16, O[e]);
            }
        }
        if (n + 1 < a.nc) preload(buf ^ 1);
    }
    __syncthreads();

    if (MODE == 0 && a.s_final) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4) =
                        make_float4(S[i][j][0], S[i][j][1], S[i][j][2], S[i][j][3]);
    }
}

template <int D, int CS>
struct Dh2Layout {
    static constexpr int DC = D / CS, PS = 8;
    static constexpr int LDR = D + PS, LDU = DC + PS, LDC = C + PS;
    static constexpr int AQKT_OFF = 0;
    static constexpr int KB_OFF = AQKT_OFF + C * LDC;
    static constexpr int QPT_OFF = KB_OFF + C * LDR;
    static constexpr int WT_OFF = QPT_OFF + D * LDC;
    static constexpr int DOT_OFF = WT_OFF + D * LDC;              // dO^T of the owned columns [DC][LDC]
    static constexpr int SET_ELEMS = DOT_OFF + DC * LDC;
    static constexpr int EG_BYTE = SET_ELEMS * 2;
    static constexpr int SET_BYTES = (EG_BYTE + D * 4 + 15) & ~15;
    static constexpr int XS_OFF = 2 * SET_BYTES;                 // dS^T  [DC][LDR]
    static constexpr int XV_OFF = XS_OFF + DC * LDR * 2;         // -dV'^T [DC][LDC]
    static constexpr int STG_OFF = XV_OFF + DC * LDC * 2;
    static constexpr int STG_ELEMS = D * LDU + C * LDU;          // dh, dV'
    static constexpr int STG_BYTES = (STG_ELEMS * 2 + 15) & ~15;
    static constexpr int NSTG = 3;                              // staging tiles, by step % 3
    static constexpr int BYTES = STG_OFF + NSTG * STG_BYTES;
    static_assert(BYTES <= 160 * 1024, "reverse recurrence LDS");
};

template <int D, int CS>
struct Dh2Slabs {
    static constexpr int DC = D / CS;
    Tile<uint16_t, C, C> AqkT;
    Tile<uint16_t, C, D> Kb;
    Tile<uint16_t, D, C> QpT, WT;
    Tile<uint16_t, C, DC> dO;
    Tile<float, 1, D> eG;
};

// Reverse state recurrence, same roles and barriers as kda_recur2_kernel:
//   compute: [A] dV' = Aqk^T dO + Kb dS (row block w), write -dV'^T [B]
//            dS <- diag(e^G) dS + Qp^T dO - W^T dV', write dS^T (and dS, the
//            chunk-end adjoint, to staging) for the next chunk
//   memory:  [A] flush [B] commit / load (dO lands transposed: dO^T[col][t])
template <int D, int CS>
__global__ __launch_bounds__(512) void kda_dh2_kernel(const DhArgs a) {
    using ST = uint16_t;
    using Lay = Dh2Layout<D, CS>;
    using Slabs = Dh2Slabs<D, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, MT = (NT + 3) / 4;
    constexpr int LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC;
    __shared__ __align__(16) unsigned char smem[Lay::BYTES];

    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lb / CS, c0 = (lb - bh * CS) * DC;
    const int b = bh / a.H, h = bh - b * a.H;

    auto set = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + buf * Lay::SET_BYTES); };
    auto seg = [&](int buf) __attribute__((always_inline)) { return reinterpret_cast<float*>(smem + buf * Lay::SET_BYTES + Lay::EG_BYTE); };
    auto stg = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<ST*>(smem + Lay::STG_OFF + sb * Lay::STG_BYTES); };
    ST* xs = reinterpret_cast<ST*>(smem + Lay::XS_OFF);
    ST* xv = reinterpret_cast<ST*>(smem + Lay::XV_OFF);

    if (wv >= 4) {
        // ---------------- memory waves ----------------
        const int mt = tid - 256;
        auto issue = [&](int n, Slabs& p) __attribute__((always_inline)) {
            const size_t ch = (size_t)bh * a.nc + n;
            const int t0 = n * C, valid = min(C, a.T - t0);
            p.AqkT.load_at(mt, static_cast<const ST*>(a.AqkT) + ch * C * C, C);
            p.Kb.load_at(mt, static_cast<const ST*>(a.Kb) + ch * C * D, D);
            p.QpT.load_at(mt, static_cast<const ST*>(a.QpT) + ch * C * D, C);
            p.WT.load_at(mt, static_cast<const ST*>(a.WT) + ch * C * D, C);
            p.eG.load_at(mt, a.eG + ch * D, D);
            p.dO.load_at(mt, static_cast<const ST*>(a.dout) + (((size_t)b * a.T + t0) * a.H + h) * D + c0,
                         (size_t)a.H * D, valid);
        };
        auto commit = [&](int buf, const Slabs& p) __attribute__((always_inline)) {
            p.AqkT.store_at(mt, set(buf) + Lay::AQKT_OFF, LDC);
            p.Kb.store_at(mt, set(buf) + Lay::KB_OFF, LDR);
            p.QpT.store_at(mt, set(buf) + Lay::QPT_OFF, LDC);
            p.WT.store_at(mt, set(buf) + Lay::WT_OFF, LDC);
            p.eG.store_at(mt, seg(buf), D);
            ST* dot = set(buf) + Lay::DOT_OFF;
            constexpr int EPV = 8, VPR = DC / EPV, NV = C * VPR;
#pragma unroll
            for (int i = 0; i < Tile<ST, C, DC>::PER; ++i) {
                const int v = mt + 256 * i;
                if (NV % 256 == 0 || v < NV) {
                    const int t = v / VPR, c = (v - t * VPR) * EPV;
                    const uint4 x = p.dO.get(i);
                    const uint32_t u[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dot[(c + 2 * e) * LDC + t] = (ST)(u[e] & 0xffffu);
                        dot[(c + 2 * e + 1) * LDC + t] = (ST)(u[e] >> 16);
                    }
                }
            }
        };
        auto flush = [&](int it, int n) __attribute__((always_inline)) {
            const ST* sst = stg(it % Lay::NSTG);
            const size_t ch = (size_t)bh * a.nc + n;
            tile_out_at<ST, D, DC>(mt, sst, LDU, static_cast<ST*>(a.dh) + ch * D * D + c0, D, D);
            tile_out_at<ST, C, DC>(mt, sst + D * LDU, LDU, static_cast<ST*>(a.dVp) + ch * C * D + c0, D, C);
        };
        // Loop step k handles chunk nc-1-k; step k's slabs live in register set
        // k % 3 from their load (three steps ahead) to their commit into LDS set
        // k & 1 (one step ahead).  Unrolled three times, as in kda_recur2_kernel.
        Slabs p0, p1, p2;
        const int nc = a.nc;
        issue(nc - 1, p0);
        if (nc > 1) issue(nc - 2, p1);
        if (nc > 2) issue(nc - 3, p2);
        commit(0, p0);
        if (nc > 3) issue(nc - 4, p0);
        __syncthreads();                                       // P: step 0 committed
        auto step = [&](int it, Slabs& p) __attribute__((always_inline)) {   // p holds step it+1
            const int n = nc - 1 - it;
            __syncthreads();                                   // A(it)
            if (it + 1 < nc) commit((it + 1) & 1, p);
            __syncthreads();                                   // B(it): step it+1 committed
            if (it > 0) flush(it - 1, n + 1);
            if (it + 4 < nc) issue(nc - 1 - (it + 4), p);
        };
        for (int it = 0; it < nc; it += 3) {
            step(it, p1);
            if (it + 1 < nc) step(it + 1, p2);
            if (it + 2 < nc) step(it + 2, p0);
        }
        __syncthreads();
        flush(nc - 1, 0);
        return;
    }

    // ---------------- compute waves ----------------
    const int w = wv, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    int mt[MT];
    bool own[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        mt[i] = w + 4 * i;
        own[i] = mt[i] < NT;
    }
    f32x4 dS[MT][NTW];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            dS[i][j] = zero4();
            if (own[i] && a.dsf) {
                const float4 x = *reinterpret_cast<const float4*>(
                    a.dsf + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4);
                dS[i][j] = f32x4{x.x, x.y, x.z, x.w};
            }
        }
    // dS^T for the B operands, dS (the chunk-end adjoint) to staging
    auto put_state = [&](ST* sst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    *reinterpret_cast<uint2*>(xs + (BS * j + r16) * LDR + BS * mt[i] + 4 * g4) = pack4bf(dS[i][j]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        st1<ST>(sst + (BS * mt[i] + 4 * g4 + e) * LDU + BS * j + r16, dS[i][j][e]);
                }
    };
    put_state(stg(0));

    Frag8 Aat[2], Akb[D / 32], Aqt[MT][C / 32], Awt[MT][C / 32], Bo[NTW][C / 32];
    float4 eg[MT];
    auto preload = [&](int buf) __attribute__((always_inline)) {
        const ST* sAqkT = set(buf) + Lay::AQKT_OFF;
        const ST* sKb = set(buf) + Lay::KB_OFF;
        const ST* sQpT = set(buf) + Lay::QPT_OFF;
        const ST* sWT = set(buf) + Lay::WT_OFF;
        const ST* sdOT = set(buf) + Lay::DOT_OFF;
        const float* seG = seg(buf);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            if (ks >= w / 2) Aat[ks] = ldfrag<1, ST>(sAqkT, LDC, BS * w, 32 * ks);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) Akb[ks] = ldfrag<1, ST>(sKb, LDR, BS * w, 32 * ks);
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bo[j][ks] = ldfrag<1, ST>(sdOT, LDC, BS * j, 32 * ks);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) {
                    Aqt[i][ks] = ldfrag<1, ST>(sQpT, LDC, BS * mt[i], 32 * ks);
                    Awt[i][ks] = ldfrag<1, ST>(sWT, LDC, BS * mt[i], 32 * ks);
                }
                eg[i] = *reinterpret_cast<const float4*>(seG + BS * mt[i] + 4 * g4);
            }
    };
    __syncthreads();                                           // P
    preload(0);

    for (int it = 0; it < a.nc; ++it) {
        const int n = a.nc - 1 - it;
        const int buf = it & 1;
        ST* sst = stg(it % Lay::NSTG);
        __syncthreads();                                       // A(it)

        Frag8 Bs[NTW][D / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = ldfrag<1, ST>(xs, LDR, BS * j, 32 * ks);
        // dV' = Aqk^T dO + Kb dS, row block w
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            f32x4 dV = zero4();
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (ks >= w / 2) dV = mma<1>(Aat[ks], Bo[j][ks], dV);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) dV = mma<1>(Akb[ks], Bs[j][ks], dV);
            *reinterpret_cast<uint2*>(xv + (BS * j + r16) * LDC + BS * w + 4 * g4) = pack4bf(negacc(dV));
#pragma unroll
            for (int e = 0; e < 4; ++e) st1<ST>(sst + D * LDU + (BS * w + 4 * g4 + e) * LDU + BS * j + r16, dV[e]);
        }
        __syncthreads();                                       // B(it)

        Frag8 Bvn[NTW][C / 32];    // -dV'
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bvn[j][ks] = ldfrag<1, ST>(xv, LDC, BS * j, 32 * ks);
        // dS <- diag(e^G) dS + Qp^T dO - W^T dV'
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    dS[i][j] = f32x4{dS[i][j][0] * eg[i].x, dS[i][j][1] * eg[i].y, dS[i][j][2] * eg[i].z,
                                     dS[i][j][3] * eg[i].w};
#pragma unroll
                    for (int ks = 0; ks < C / 32; ++ks) {
                        dS[i][j] = mma<1>(Awt[i][ks], Bvn[j][ks], dS[i][j]);
                        dS[i][j] = mma<1>(Aqt[i][ks], Bo[j][ks], dS[i][j]);
                    }
                }
            }
        if (n > 0) {
            put_state(stg((it + 1) % Lay::NSTG));
            preload(buf ^ 1);
        }
    }
    __syncthreads();

    if (a.ds0) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<float4*>(a.ds0 + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4) =
                        make_float4(dS[i][j][0], dS[i][j][1], dS[i][j][2], dS[i][j][3]);
    }
}

// ----------------------------------------------------------------------------
// bf16 recurrences, row split, LDS-DMA fed (kda_recur3_kernel; the reverse
// carry kda_dh4_kernel below uses the same slab sets, Dh3Layout).
//
// CS workgroups per (batch, head) own DC = D / CS state columns each.  Wave w
// owns row block w of the chunk's [C][DC] tiles and state row blocks w, w + 4.
// The chunk slabs reach LDS by DMA (no registers, no commit step) into NS
// swizzled LDS sets, NS chunks ahead; each chunk's A operands are read into
// registers one chunk ahead, so after a barrier only the exchanged state / V'
// fragments are read.  Per chunk n:
//   A(n)  flush chunk n-1's staged outputs; DMA chunk n+NS into set n % NS;
//         V' = U - W S (row block w); write V'^T; wait for chunk n+1's DMA
//   B(n)  S <- diag(e^G) S + Kb^T V' (own state rows); write S^T for chunk n+1;
//         O = Qp S + Aqk V' -> staging; read chunk n+1's A operands
// Barriers are lds_barrier(): DMA stays in flight across them, and each wave
// waits with an explicit vmcnt for exactly the DMA it needs.
// MODE 0 writes O and the final state, MODE 1 the chunk-start states h.
// ----------------------------------------------------------------------------
template <int D, int MODE, int CS>
struct Recur3Layout {
    static constexpr int DC = D / CS, NS = (D >= 128) ? 2 : 3;
    static constexpr int RB_W = 2 * D, RB_U = 2 * DC, RB_C = 2 * C;          // swizzled row bytes
    static constexpr int W_OFF = 0;                                           // [C][D]
    static constexpr int U_OFF = W_OFF + C * RB_W;                            // [C][DC]
    static constexpr int QP_OFF = U_OFF + C * RB_U;                           // [C][D]   (MODE 0)
    static constexpr int KBT_OFF = QP_OFF + (MODE == 0 ? C * RB_W : 0);        // Kb^T [D][C] (recur3), Kb [C][D] (recur4)
    static constexpr int AQK_OFF = KBT_OFF + D * RB_C;                        // [C][C]   (MODE 0)
    static constexpr int EG_OFF = AQK_OFF + (MODE == 0 ? C * RB_C : 0);        // [D] fp32
    static constexpr int SET_BYTES = (EG_OFF + 4 * D + 1023) & ~1023;
    // Staging rows (LDU) keep a 16-byte pad for 16-byte row access.  The
    // exchange tiles (LDR, LDC) are only touched 8 bytes at a time: a 4-element
    // pad (rows of 34 dwords, 2 mod 32) puts the 16 rows of a fragment read or
    // a C-layout write in 16 distinct bank pairs.
    static constexpr int PS = 8, PX = 4, LDR = D + PX, LDU = DC + PS, LDC = C + PX;
    // exchange and staging live in a __shared__ array of their own
    static constexpr int XS_OFF = 0;                                          // S^T  [DC][LDR] bf16
    static constexpr int XV_OFF = XS_OFF + DC * LDR * 2;                      // V'^T [DC][LDC] bf16
    static constexpr int STG_OFF = XV_OFF + DC * LDC * 2;
    static constexpr int STG_ELEMS = (MODE == 0) ? C * LDU : D * LDU;   // O | h
    static constexpr int STG_BYTES = (STG_ELEMS * 2 + 15) & ~15;
    // h for chunk n+1 is staged while chunk n-1 is flushed: three tiles
    static constexpr int NSTG = (MODE == 0) ? 2 : 3;
    static constexpr int XBYTES = STG_OFF + NSTG * STG_BYTES;
    static_assert(NS * SET_BYTES + XBYTES <= 160 * 1024, "recurrence LDS");
    // DMA wave-instructions per wave per chunk
    static constexpr int L = DmaTile<C, RB_W, 4>::COUNT + DmaTile<C, RB_U, 4>::COUNT + DmaTile<D, RB_C, 4>::COUNT +
                             (MODE == 0 ? DmaTile<C, RB_W, 4>::COUNT + DmaTile<C, RB_C, 4>::COUNT : 0) + 1;
};


template <int D, int MODE, int CS>
__global__ __launch_bounds__(256) void kda_recur3_kernel(const RecurArgs a) {
    using ST = uint16_t;
    using Lay = Recur3Layout<D, MODE, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, MT = (NT + 3) / 4, NS = Lay::NS;
    constexpr int LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC;
    constexpr int RB_W = Lay::RB_W, RB_U = Lay::RB_U, RB_C = Lay::RB_C;
    __shared__ __align__(1024) char set0[Lay::SET_BYTES];
    __shared__ __align__(1024) char set1[Lay::SET_BYTES];
    __shared__ __align__(1024) char set2[NS == 3 ? Lay::SET_BYTES : 16];
    __shared__ __align__(16) char smem[Lay::XBYTES];

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, g4 = l >> 4;
    __builtin_assume(w >= 0 && w < 4);
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lb / CS, c0 = (lb - bh * CS) * DC;
    const int b = bh / a.H, h = bh - b * a.H;
    const int nc = a.nc;
    const char* gW = static_cast<const char*>(a.W);
    const char* gU = static_cast<const char*>(a.U);
    const char* gQp = static_cast<const char*>(a.Qp);
    const char* gKbT = static_cast<const char*>(a.KbT);
    const char* gAqk = static_cast<const char*>(a.Aqk);
    const char* gEg = reinterpret_cast<const char*>(a.eG);

    auto stg = [&](int c) __attribute__((always_inline)) {
        return reinterpret_cast<ST*>(smem + Lay::STG_OFF + (c % Lay::NSTG) * Lay::STG_BYTES);
    };
    ST* xs = reinterpret_cast<ST*>(smem + Lay::XS_OFF);
    ST* xv = reinterpret_cast<ST*>(smem + Lay::XV_OFF);

    // chunk c's slabs -> LDS set sb = set (c % NS) (Lay::L instructions per wave)
    using TW = DmaTile<C, RB_W, 4>;
    using TU = DmaTile<C, RB_U, 4>;
    using TK = DmaTile<D, RB_C, 4>;
    using TA = DmaTile<C, RB_C, 4>;
    uint32_t oW[TW::COUNT], oU[TU::COUNT], oK[TK::COUNT], oA[TA::COUNT];
    TW::offsets(oW, RB_W, w, l);
    TU::offsets(oU, (size_t)D * 2, w, l);
    TK::offsets(oK, RB_C, w, l);
    TA::offsets(oA, RB_C, w, l);
    const uint32_t oE = (uint32_t)((D / 4) * 4 * w + 16 * (l < D / 16 ? l : 0));
    auto dma_chunk = [&](int c, char* sb) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * nc + c;
        TW::issue_s(gW + ch * C * D * 2, oW, sb + Lay::W_OFF, w);
        TU::issue_s(gU + (ch * C * D + c0) * 2, oU, sb + Lay::U_OFF, w);
        TK::issue_s(gKbT + ch * C * D * 2, oK, sb + Lay::KBT_OFF, w);
        if constexpr (MODE == 0) {
            TW::issue_s(gQp + ch * C * D * 2, oW, sb + Lay::QP_OFF, w);
            TA::issue_s(gAqk + ch * C * C * 2, oA, sb + Lay::AQK_OFF, w);
        }
        // e^G: D floats, D / 16 lanes of 16 bytes per wave
        if (l < D / 16) dma16_s(gEg + ch * D * 4, oE, sb + Lay::EG_OFF + D * w);
    };
    auto flush = [&](int n) __attribute__((always_inline)) {
        const ST* sst = stg(n);
        if constexpr (MODE == 0) {
            const int t0 = n * C, valid = min(C, a.T - t0);
            tile_out<ST, C, DC>(sst, LDU, static_cast<ST*>(a.o) + (((size_t)b * a.T + t0) * a.H + h) * D + c0,
                                (size_t)a.H * D, valid);
        } else {
            const size_t ch = (size_t)bh * nc + n;
            tile_out<ST, D, DC>(sst, LDU, static_cast<ST*>(a.h) + ch * D * D + c0, D, D);
        }
    };

    int mt[MT];
    bool own[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        mt[i] = w + 4 * i;
        own[i] = mt[i] < NT;
    }
    f32x4 S[MT][NTW];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            S[i][j] = zero4();
            if (own[i] && a.s0) {
                const float4 x = *reinterpret_cast<const float4*>(
                    a.s0 + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4);
                S[i][j] = f32x4{x.x, x.y, x.z, x.w};
            }
        }
    // S^T for the B operands (and, for the backward, the chunk-start state)
    auto put_state = [&](ST* sst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    *reinterpret_cast<uint2*>(xs + (BS * j + r16) * LDR + BS * mt[i] + 4 * g4) = pack4bf(S[i][j]);
                    if constexpr (MODE == 1)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            st1<ST>(sst + (BS * mt[i] + 4 * g4 + e) * LDU + BS * j + r16, S[i][j][e]);
                }
    };

    // one chunk's A operands, read ahead from its LDS set
    Frag8 Aw[D / 32], Aq[D / 32], Aa[2], Akb[MT][C / 32];
    f32x4 Uv[NTW];
    float4 eg[MT];
    auto preload = [&](const char* sb) __attribute__((always_inline)) {
        const ST* sW = reinterpret_cast<const ST*>(sb + Lay::W_OFF);
        const ST* sU = reinterpret_cast<const ST*>(sb + Lay::U_OFF);
        const ST* sKbT = reinterpret_cast<const ST*>(sb + Lay::KBT_OFF);
        const float* seG = reinterpret_cast<const float*>(sb + Lay::EG_OFF);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) Aw[ks] = ldfrag_sw<RB_W>(sW, BS * w, 32 * ks);
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) Uv[j][e] = ld_sw<RB_U>(sU, BS * w + 4 * g4 + e, BS * j + r16);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) Akb[i][ks] = ldfrag_sw<RB_C>(sKbT, BS * mt[i], 32 * ks);
                eg[i] = *reinterpret_cast<const float4*>(seG + BS * mt[i] + 4 * g4);
            }
        if constexpr (MODE == 0) {
            const ST* sQp = reinterpret_cast<const ST*>(sb + Lay::QP_OFF);
            const ST* sAqk = reinterpret_cast<const ST*>(sb + Lay::AQK_OFF);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Aq[ks] = ldfrag_sw<RB_W>(sQp, BS * w, 32 * ks);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (ks <= w / 2) Aa[ks] = ldfrag_sw<RB_C>(sAqk, BS * w, 32 * ks);
        }
    };

    // prologue: chunks 0 .. NS-1 in flight, chunk 0 landed and read
    put_state(stg(0));
    dma_chunk(0, set0);
    if (nc > 1) dma_chunk(1, set1);
    if (NS == 3 && nc > 2) dma_chunk(2, set2);
    dma_wait_chunks<Lay::L>(min(NS, nc) - 1);
    lds_barrier();
    preload(set0);

    // chunk n: DMA chunk n+NS into sdma (set n % NS), read chunk n+1's A
    // operands from snext (set (n+1) % NS)
    auto step = [&](int n, char* sdma, const char* snext) __attribute__((always_inline)) {
        ST* sst = stg(n);
        lds_barrier();                                          // A(n)
        if (n > 0) flush(n - 1);
        if (n + NS < nc) dma_chunk(n + NS, sdma);

        Frag8 Bs[NTW][D / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = ldfrag<1, ST>(xs, LDR, BS * j, 32 * ks);
        // V' = U - W S, row block w
        f32x4 Vp[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            f32x4 P = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) P = mma<1>(Aw[ks], Bs[j][ks], P);
#pragma unroll
            for (int e = 0; e < 4; ++e) Vp[j][e] = Uv[j][e] - P[e];
            *reinterpret_cast<uint2*>(xv + (BS * j + r16) * LDC + BS * w + 4 * g4) = pack4bf(Vp[j]);
        }
        // chunk n+1's DMA (this wave's share) complete; later chunks may stay in flight
        dma_wait_chunks<Lay::L>(min(nc - 1, n + NS) - (n + 1));
        lds_barrier();                                          // B(n)

        Frag8 Bv[NTW][C / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bv[j][ks] = ldfrag<1, ST>(xv, LDC, BS * j, 32 * ks);
        // S <- diag(e^G) S + Kb^T V'
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    S[i][j] = f32x4{S[i][j][0] * eg[i].x, S[i][j][1] * eg[i].y, S[i][j][2] * eg[i].z,
                                    S[i][j][3] * eg[i].w};
#pragma unroll
                    for (int ks = 0; ks < C / 32; ++ks) S[i][j] = mma<1>(Akb[i][ks], Bv[j][ks], S[i][j]);
                }
            }
        if (n + 1 < nc) put_state(stg(n + 1));
        if constexpr (MODE == 0) {
            // O = Qp S + Aqk V', row block w (the chunk-start state is in Bs)
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                f32x4 O = zero4();
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) O = mma<1>(Aq[ks], Bs[j][ks], O);
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    if (ks <= w / 2) O = mma<1>(Aa[ks], Bv[j][ks], O);
#pragma unroll
                for (int e = 0; e < 4; ++e) st1<ST>(sst + (BS * w + 4 * g4 + e) * LDU + BS * j + r16, O[e]);
            }
        }
        if (n + 1 < nc) preload(snext);
    };
    // unrolled NS times so that every set is named statically
    for (int n = 0; n < nc; n += NS) {
        step(n, set0, set1);
        if (n + 1 < nc) step(n + 1, set1, NS == 3 ? set2 : set0);
        if (NS == 3 && n + 2 < nc) step(n + 2, set2, set0);
    }
    lds_barrier();
    flush(nc - 1);

    if (MODE == 0 && a.s_final) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4) =
                        make_float4(S[i][j][0], S[i][j][1], S[i][j][2], S[i][j][3]);
    }
}

// ----------------------------------------------------------------------------
// kda_recur4_kernel: kda_recur3_kernel with the per-chunk work split between
// two wave roles, so that one wave per SIMD runs the state chain while the
// other does the work off it.  512 threads; role 0 = waves 0-3 (chain), role 1
// = waves 4-7.  Wave wr = w % 4 of a role owns row block wr of the chunk tiles.
//   chain waves: V' = U - W S (row block wr), write V'^T; after B: state update
//                of state rows wr, wr + 4, write S^T (MODE 1: and h); read the
//                next chunk's W, U, Kb^T (transposing reads of Kb), e^G operands
//   role-1 waves: flush the previous chunk's outputs; MODE 0: O = Qp S + Aqk V'
//                (row block wr) after B, read the next chunk's Qp, Aqk operands;
//                MODE 1: copy the chunk-start state to h
//   DMA: chunk n+NS is brought after barrier B(n), once chunk n's operands (the
//        chain waves read its Kb^T and e^G between A(n) and B(n)) have left its
//        LDS set: MODE 0 the chain waves bring W, U, Kb^T, e^G after their state
//        update and the role-1 waves Qp, Aqk; MODE 1 the role-1 waves bring all.
// The barriers, LDS sets and staging are those of kda_recur3_kernel.
// ----------------------------------------------------------------------------
template <int D, int MODE, int CS>
__global__ __launch_bounds__(512) void kda_recur4_kernel(const RecurArgs a) {
    using ST = uint16_t;
    constexpr bool FWD = MODE == 0;   // O and the final state
    using Lay = Recur3Layout<D, FWD ? 0 : 1, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, MT = (NT + 3) / 4, NS = Lay::NS;
    constexpr int LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC;
    constexpr int RB_W = Lay::RB_W, RB_U = Lay::RB_U, RB_C = Lay::RB_C;
    __shared__ __align__(1024) char set0[Lay::SET_BYTES];
    __shared__ __align__(1024) char set1[Lay::SET_BYTES];
    __shared__ __align__(1024) char set2[NS == 3 ? Lay::SET_BYTES : 16];
    __shared__ __align__(16) char smem[Lay::XBYTES];

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, g4 = l >> 4;
    __builtin_assume(w >= 0 && w < 8);
    const int role = w >> 2, wr = w & 3;
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lb / CS, c0 = (lb - bh * CS) * DC;
    const int b = bh / a.H, h = bh - b * a.H;
    const int nc = a.nc;
    const char* gW = static_cast<const char*>(a.W);
    const char* gU = static_cast<const char*>(a.U);
    const char* gQp = static_cast<const char*>(a.Qp);
    const char* gKb = static_cast<const char*>(a.Kb);
    const char* gAqk = static_cast<const char*>(a.Aqk);
    const char* gEg = reinterpret_cast<const char*>(a.eG);

    auto stg = [&](int c) __attribute__((always_inline)) {
        return reinterpret_cast<ST*>(smem + Lay::STG_OFF + (c % Lay::NSTG) * Lay::STG_BYTES);
    };
    ST* xs = reinterpret_cast<ST*>(smem + Lay::XS_OFF);
    ST* xv = reinterpret_cast<ST*>(smem + Lay::XV_OFF);

    using TW = DmaTile<C, RB_W, 4>;   // W, Kb, Qp
    using TU = DmaTile<C, RB_U, 4>;
    using TA = DmaTile<C, RB_C, 4>;
    // which role brings the state-chain slabs (W, U, Kb, e^G) and how many DMA
    // instructions per chunk this wave issues
    constexpr int CHAIN_ROLE = FWD ? 0 : 1;
    constexpr int L_CHAIN = 2 * TW::COUNT + TU::COUNT + 1;
    constexpr int L_OUT = FWD ? TW::COUNT + TA::COUNT : 0;
    constexpr int L0 = (CHAIN_ROLE == 0) ? L_CHAIN : 0;
    constexpr int L1 = ((CHAIN_ROLE == 1) ? L_CHAIN : 0) + L_OUT;
    const bool chain_dma = role == CHAIN_ROLE;
    uint32_t oW[TW::COUNT], oU[TU::COUNT], oA[TA::COUNT];
    TW::offsets(oW, RB_W, wr, l);
    TU::offsets(oU, (size_t)D * 2, wr, l);
    TA::offsets(oA, RB_C, wr, l);
    const uint32_t oE = (uint32_t)((D / 4) * 4 * wr + 16 * (l < D / 16 ? l : 0));
    auto dma_chunk = [&](int c, char* sbp) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * nc + c;
        const uint32_t sb = lds_addr(sbp);
        if (chain_dma) {
            TW::issue_s32(gW + ch * C * D * 2, oW, sb + Lay::W_OFF, wr);
            TU::issue_s32(gU + (ch * C * D + c0) * 2, oU, sb + Lay::U_OFF, wr);
            TW::issue_s32(gKb + ch * C * D * 2, oW, sb + Lay::KBT_OFF, wr);   // Kb, [C][D]
            if (l < D / 16) dma16_s32(gEg + ch * D * 4, oE, sb + Lay::EG_OFF + D * wr);
        }
        if constexpr (FWD) {
            if (role == 1) {
                TW::issue_s32(gQp + ch * C * D * 2, oW, sb + Lay::QP_OFF, wr);
                TA::issue_s32(gAqk + ch * C * C * 2, oA, sb + Lay::AQK_OFF, wr);
            }
        }
    };
    // this wave's DMA of all but the last k chunks in flight complete
    auto dma_wait_own = [&](int k) __attribute__((always_inline)) {
        if (role == 0) {
            if constexpr (L0 > 0) dma_wait_chunks<L0>(k);
        } else {
            if constexpr (L1 > 0) dma_wait_chunks<L1>(k);
        }
    };
    // MODE 0: O of chunk n is staged transposed, O^T [DC][LDO] (a lane's four
    // rows of one column are one 8-byte write), and flushed by the role-1 waves
    // as 16-byte row pieces by transposing reads
    constexpr int LDO = C + 4;
    static_assert(DC * LDO * 2 <= Lay::STG_BYTES, "O^T staging fits a staging tile");
    auto flush = [&](int n) __attribute__((always_inline)) {   // role-1 waves
        static_assert(DC == 32 && C * DC / 8 == 256, "one 16-byte piece of O per role-1 thread");
        const int t1 = tid - 256, i = t1 & 15, row = 4 * (t1 >> 4) + (i & 3), col = 8 * (i >> 2);
        const int t0 = n * C, valid = min(C, a.T - t0);
        const short8v x = ld_tr_rows8(stg(n), LDO, 0, 4 * (t1 >> 4));
        if (row < valid)
            *reinterpret_cast<short8v*>(static_cast<ST*>(a.o) + (((size_t)b * a.T + t0 + row) * a.H + h) * D + c0 +
                                        col) = x;
    };
    // MODE 1, role-1 waves: h of chunk n is the state in xs (S^T, there between
    // A(n) and B(n)), copied to global as 16-byte row pieces of h by
    // transposing reads, so the chain waves stage nothing for it
    auto copy_h = [&](int n) __attribute__((always_inline)) {
        static_assert(DC == 32 && D * DC / 8 == 256, "one 16-byte piece of h per role-1 thread");
        const int t1 = tid - 256, i = t1 & 15, row = 4 * (t1 >> 4) + (i & 3), col = 8 * (i >> 2);
        const short8v x = ld_tr_rows8(xs, LDR, 0, 4 * (t1 >> 4));
        *reinterpret_cast<short8v*>(static_cast<ST*>(a.h) + ((size_t)bh * nc + n) * D * D + (size_t)row * D + c0 +
                                    col) = x;
    };

    int mt[MT];
    bool own[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        mt[i] = wr + 4 * i;
        own[i] = role == 0 && mt[i] < NT;
    }
    f32x4 S[MT][NTW];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            S[i][j] = zero4();
            if (own[i] && a.s0) {
                const float4 x = *reinterpret_cast<const float4*>(
                    a.s0 + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4);
                S[i][j] = f32x4{x.x, x.y, x.z, x.w};
            }
        }
    // S^T for the B operands (and, for MODE 1, the copy to h)
    auto put_state = [&]() __attribute__((always_inline)) {   // chain waves
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<uint2*>(xs + (BS * j + r16) * LDR + BS * mt[i] + 4 * g4) = pack4bf(S[i][j]);
    };

    // one chunk's A operands, read ahead from its LDS set (each role its own)
    Frag8 Aw[D / 32], Aq[D / 32], Aa[2], Akb[MT][C / 32];
    f32x4 Ov[NTW];   // role 1, MODE 0: the chunk's Qp S part of O, across barrier B
    f32x4 Uv[NTW];
    float4 eg[MT];
    // chain waves: the state-update operands (Kb^T rows, e^G) of a chunk, read
    // after its V' is out (they are needed only after barrier B)
    auto preload_kb = [&](const char* sb) __attribute__((always_inline)) {
        const ST* sKbT = reinterpret_cast<const ST*>(sb + Lay::KBT_OFF);
        const float* seG = reinterpret_cast<const float*>(sb + Lay::EG_OFF);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) Akb[i][ks] = ldfragT_sw<RB_W>(sKbT, BS * mt[i], 32 * ks);
                eg[i] = *reinterpret_cast<const float4*>(seG + BS * mt[i] + 4 * g4);
            }
    };
    auto preload = [&](const char* sb) __attribute__((always_inline)) {
        if (role == 0) {
            const ST* sW = reinterpret_cast<const ST*>(sb + Lay::W_OFF);
            const ST* sU = reinterpret_cast<const ST*>(sb + Lay::U_OFF);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Aw[ks] = ldfrag_sw<RB_W>(sW, BS * wr, 32 * ks);
#pragma unroll
            for (int j = 0; j < NTW; ++j) Uv[j] = ld_col4_sw<RB_U>(sU, BS * j, BS * wr);
        } else if constexpr (FWD) {
            const ST* sQp = reinterpret_cast<const ST*>(sb + Lay::QP_OFF);
            const ST* sAqk = reinterpret_cast<const ST*>(sb + Lay::AQK_OFF);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Aq[ks] = ldfrag_sw<RB_W>(sQp, BS * wr, 32 * ks);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (ks <= wr / 2) Aa[ks] = ldfrag_sw<RB_C>(sAqk, BS * wr, 32 * ks);
        }
    };

    // prologue: chunks 0 .. NS-1 in flight, chunk 0 landed and read
    if (role == 0) put_state();
    dma_chunk(0, set0);
    if (nc > 1) dma_chunk(1, set1);
    if (NS == 3 && nc > 2) dma_chunk(2, set2);
    dma_wait_own(min(NS, nc) - 1);
    lds_barrier();
    preload(set0);

    auto step = [&](int n, char* sdma, const char* snext, const char* scur) __attribute__((always_inline)) {
        ST* sst = stg(n);
        lds_barrier();                                          // A(n): S^T of chunk n in xs
        Frag8 Bs[NTW][D / 32];
        if (role == 0 || FWD) {
#pragma unroll
            for (int j = 0; j < NTW; ++j)
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = ldfrag<1, ST>(xs, LDR, BS * j, 32 * ks);
        }
        if (role == 0) {
            // V' = U - W S, row block wr
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                f32x4 P = zero4();
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) P = mma<1>(Aw[ks], Bs[j][ks], P);
                f32x4 Vp;
#pragma unroll
                for (int e = 0; e < 4; ++e) Vp[e] = Uv[j][e] - P[e];
                *reinterpret_cast<uint2*>(xv + (BS * j + r16) * LDC + BS * wr + 4 * g4) = pack4bf(Vp);
            }
            preload_kb(scur);
        } else if constexpr (FWD) {
            // O = Qp S + Aqk V': the Qp S part now, from the chunk-start state
            // (beside the chain's V'), the Aqk V' part after barrier B
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                Ov[j] = zero4();
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) Ov[j] = mma<1>(Aq[ks], Bs[j][ks], Ov[j]);
            }
            if (n > 0) flush(n - 1);
        } else {
            copy_h(n);
        }
        // chunk n+1's slabs landed; chunks up to n+NS-1 (issued after earlier B
        // barriers) may stay in flight
        dma_wait_own(min(nc - 1, n + NS - 1) - (n + 1));
        lds_barrier();                                          // B(n): V'^T in xv, chunk n+1 visible
        // set n % NS is free now (chunk n's operands are all in registers); the
        // chain waves bring their share after the state update
        if (role == 1 && n + NS < nc) dma_chunk(n + NS, sdma);

        Frag8 Bv[NTW][C / 32];
        if (role == 0 || FWD) {
#pragma unroll
            for (int j = 0; j < NTW; ++j)
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) Bv[j][ks] = ldfrag<1, ST>(xv, LDC, BS * j, 32 * ks);
        }
        if (role == 0) {
            // S <- diag(e^G) S + Kb^T V'
#pragma unroll
            for (int i = 0; i < MT; ++i)
                if (own[i]) {
#pragma unroll
                    for (int j = 0; j < NTW; ++j) {
                        S[i][j] = f32x4{S[i][j][0] * eg[i].x, S[i][j][1] * eg[i].y, S[i][j][2] * eg[i].z,
                                        S[i][j][3] * eg[i].w};
#pragma unroll
                        for (int ks = 0; ks < C / 32; ++ks) S[i][j] = mma<1>(Akb[i][ks], Bv[j][ks], S[i][j]);
                    }
                }
            if (n + 1 < nc) put_state();
            if (n + NS < nc) dma_chunk(n + NS, sdma);
        } else if constexpr (FWD) {
            // O += Aqk V', row block wr; staged as O^T
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                f32x4 O = Ov[j];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    if (ks <= wr / 2) O = mma<1>(Aa[ks], Bv[j][ks], O);
                *reinterpret_cast<uint2*>(sst + (BS * j + r16) * LDO + BS * wr + 4 * g4) = pack4bf(O);
            }
        }
        if (n + 1 < nc) preload(snext);
    };
    // unrolled NS times so that every set is named statically
    for (int n = 0; n < nc; n += NS) {
        step(n, set0, set1, set0);
        if (n + 1 < nc) step(n + 1, set1, NS == 3 ? set2 : set0, set1);
        if (NS == 3 && n + 2 < nc) step(n + 2, set2, set0, set2);
    }
    lds_barrier();
    if (FWD && role == 1) flush(nc - 1);

    if (FWD && a.s_final) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4) =
                        make_float4(S[i][j][0], S[i][j][1], S[i][j][2], S[i][j][3]);
    }
}

// ----------------------------------------------------------------------------
// kda_recur5_kernel: the bf16 forward recurrence with one 16-wave workgroup per
// (batch, head), so that every output row is whole inside one workgroup and the
// flush can apply the layer's gated RMSNorm (EPI):
//   y = o rsqrt(mean_d o^2 + eps) w sigmoid(z)
// (RMSNormGated, nope_gdn_mlx.py:340-366, applied to the recurrence output at
// nope_gdn_mlx.py:880-885), storing y beside o.
//   chain waves 0-7: wave w, wr = w % 4, hf = w / 4, owns row block wr of the
//     chunk tiles and state columns DH hf .. DH hf + DH - 1 (DH = D / 2): the
//     work of a kda_recur4_kernel chain wave (V' = U - W S of its rows and
//     columns, V'^T out; after B the state update of state row block wr, S^T
//     out), and after the update the DMA of all of a later chunk's slabs.
//   side waves 8-15: wave w computes O = Qp S + Aqk V' for row block wr and
//     the columns of half hf (Qp S after A, beside the chain's V'; Aqk V' after
//     B) into the staging tile, and flushes 16 bytes of each of the previous
//     chunk's staged rows (after A; with EPI after the staging, where the
//     norm's work waits on no barrier); the eight lanes of a row are adjacent.
//     With EPI the chain waves bring the chunk's gate rows with its slabs, and
//     the side waves copy their flush pieces of them into registers before B
//     (the set is refilled after B), one register set per parity of the chunk.
//     The side waves issue no global load and no DMA: their only vector-memory
//     operations are the flush stores, so no wait of theirs can stall on a load
//     in flight.
// Barriers and wait counts follow kda_recur4_kernel; the slabs are read once
// per (batch, head) instead of once per column half.  LDS sets: NS = 3 (DMA
// three chunks ahead), with EPI NS = 2 (each set also holds the gate tile).
// ----------------------------------------------------------------------------
template <int D, bool EPI>
struct Recur5Layout {
    static constexpr int NS = EPI ? 2 : 3;
    static constexpr int RB = 2 * D, RB_C = 2 * C;                     // swizzled row bytes
    static constexpr int W_OFF = 0;                                    // [C][D]
    static constexpr int U_OFF = W_OFF + C * RB;                       // [C][D]
    static constexpr int QP_OFF = U_OFF + C * RB;                      // [C][D]
    static constexpr int KB_OFF = QP_OFF + C * RB;                     // [C][D]
    static constexpr int AQK_OFF = KB_OFF + C * RB;                    // [C][C]
    static constexpr int EG_OFF = AQK_OFF + C * RB_C;                  // [D] fp32
    static constexpr int Z_OFF = EG_OFF + 4 * D;                       // [C][D] gate rows (EPI)
    static constexpr int SET_BYTES = ((EPI ? Z_OFF + C * RB : Z_OFF) + 1023) & ~1023;
    // exchange tiles with a 4-element pad (see Recur3Layout), staging rows with 16 bytes
    static constexpr int PS = 8, PX = 4, LDR = D + PX, LDU = D + PS, LDC = C + PX;
    static constexpr int XS_OFF = 0;                                   // S^T  [D][LDR] bf16
    static constexpr int XV_OFF = XS_OFF + D * LDR * 2;                // V'^T [D][LDC] bf16
    static constexpr int STG_OFF = XV_OFF + D * LDC * 2;               // O    [C][LDU] bf16, two
    static constexpr int STG_BYTES = (C * LDU * 2 + 15) & ~15;
    static constexpr int NW_OFF = STG_OFF + 2 * STG_BYTES;            // norm weight [D] fp32
    static constexpr int XBYTES = NW_OFF + 4 * D;
    static_assert(NS * SET_BYTES + XBYTES <= 160 * 1024, "recurrence LDS");
};

template <int D, bool EPI>
__global__ __launch_bounds__(1024) void kda_recur5_kernel(const RecurArgs a) {
    using ST = uint16_t;
    using Lay = Recur5Layout<D, EPI>;
    constexpr int NS = Lay::NS, LDR = Lay::LDR, LDU = Lay::LDU, LDC = Lay::LDC, RB = Lay::RB, RB_C = Lay::RB_C;
    constexpr int DH = D / 2, NTW = DH / BS;
    static_assert(D == 64, "chain wave wr owns state row block wr: four row blocks");
    __shared__ __align__(1024) char set0[Lay::SET_BYTES];
    __shared__ __align__(1024) char set1[Lay::SET_BYTES];
    __shared__ __align__(1024) char set2[NS == 3 ? Lay::SET_BYTES : 16];
    __shared__ __align__(16) char smem[Lay::XBYTES];

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, g4 = l >> 4;
    __builtin_assume(w >= 0 && w < 16);
    const bool chain = w < 8;
    const int wr = w & 3, cb = DH * ((w >> 2) & 1);
    const int bh = xcd_remap(blockIdx.x, gridDim.x);
    const int b = bh / a.H, h = bh - b * a.H;
    const int nc = a.nc;
    const char* gW = static_cast<const char*>(a.W);
    const char* gU = static_cast<const char*>(a.U);
    const char* gQp = static_cast<const char*>(a.Qp);
    const char* gKb = static_cast<const char*>(a.Kb);
    const char* gAqk = static_cast<const char*>(a.Aqk);
    const char* gEg = reinterpret_cast<const char*>(a.eG);

    auto stg = [&](int c) __attribute__((always_inline)) {
        return reinterpret_cast<ST*>(smem + Lay::STG_OFF + (c & 1) * Lay::STG_BYTES);
    };
    ST* xs = reinterpret_cast<ST*>(smem + Lay::XS_OFF);
    ST* xv = reinterpret_cast<ST*>(smem + Lay::XV_OFF);

    // every slab tile is eight 1 KB blocks: one per chain wave
    using TR = DmaTile<C, RB, 8>;     // W, U, Qp, Kb
    using TC = DmaTile<D, RB_C, 8>;   // Aqk
    constexpr int L_CHAIN = 4 * TR::COUNT + TC::COUNT + 1 + (EPI ? 1 : 0);   // + e^G (32 B), gate rows
    static_assert(C == D && 4 * D == 8 * 32, "square tiles; e^G: two 16-byte lanes per chain wave");
    uint32_t oR[TR::COUNT], oC[TC::COUNT];
    TR::offsets(oR, RB, chain ? w : 0, l);
    TC::offsets(oC, RB_C, chain ? w : 0, l);
    const uint32_t oE = (uint32_t)(32 * w + 16 * (l & 1));
    // one chunk's slabs into an LDS set, by the chain waves after their state update
    auto dma_chunk = [&](int c, char* sbp) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * nc + c;
        const uint32_t sb = lds_addr(sbp);
        TR::issue_s32(gW + ch * C * D * 2, oR, sb + Lay::W_OFF, w);
        TR::issue_s32(gU + ch * C * D * 2, oR, sb + Lay::U_OFF, w);
        TR::issue_s32(gKb + ch * C * D * 2, oR, sb + Lay::KB_OFF, w);
        if (l < 2) dma16_s32(gEg + ch * D * 4, oE, sb + Lay::EG_OFF + 32 * w);
        TR::issue_s32(gQp + ch * C * D * 2, oR, sb + Lay::QP_OFF, w);
        TC::issue_s32(gAqk + ch * C * C * 2, oC, sb + Lay::AQK_OFF, w);
        if constexpr (EPI) {
            // the chunk's gate rows, [C][D] swizzled like the slabs: wave w's
            // 1 KB block is rows 8 w .. 8 w + 7, lane l row 8 w + l / 8 and the
            // 16-byte column piece that lands at piece l % 8 (rows past T
            // repeat the last row, so every lane issues)
            const int t0 = c * C, valid = min(C, a.T - t0);
            const int rr = 8 * w + (l >> 3), pc = (l & 7) ^ (rr & Swz<RB>::M);
            const ST* gz = static_cast<const ST*>(a.z) + ((size_t)b * a.T + t0 + min(rr, valid - 1)) * a.ld_z +
                           (size_t)h * D + 8 * pc;
            dma16(gz, sbp + Lay::Z_OFF + 1024 * w);
        }
    };

    // Registers carried from one chunk step to the next, shared by the roles:
    //   Ax: chain W rows (A of V' = U - W S), side Qp rows;
    //   Ay: chain Kb^T rows (A of the state update, transposing reads of Kb),
    //       side Aqk rows;
    //   Rx: chain U of its rows and columns, side (EPI) its flush piece of the
    //       gate rows of even chunks, as raw bits (Rz[0]: odd chunks).
    Frag8 Ax[D / 32], Ay[2];
    f32x4 Rx[NTW], Rz[1];
    float4 eg;

    // side waves: the flush thread t1 = tid - 512 owns the 16-byte piece
    // (row t1 / 8, columns 8 (t1 % 8) ..) of a staged tile
    const int t1 = tid - 512, frow = t1 >> 3, fcol = (t1 & 7) * 8;
    float* snw = reinterpret_cast<float*>(smem + Lay::NW_OFF);
    if constexpr (EPI) {
        if (!chain && t1 < D) snw[t1] = a.nw[t1];
    }
    // this thread's flush piece of a chunk's gate rows, from its LDS set
    auto read_gate = [&](const char* sb, f32x4& Z) __attribute__((always_inline)) {
        Z = __builtin_bit_cast(f32x4, *reinterpret_cast<const uint4*>(sb + Lay::Z_OFF + Swz<RB>::at(frow, 2 * fcol)));
    };
    // side waves: chunk n's staged rows (with EPI and its gate piece Z)
    auto flush = [&](int n, const f32x4& Z) __attribute__((always_inline)) {
        const ST* sst = stg(n);
        const int t0 = n * C, valid = min(C, a.T - t0);
        const uint4 ov = *reinterpret_cast<const uint4*>(sst + frow * LDU + fcol);
        ST* go = static_cast<ST*>(a.o) + (((size_t)b * a.T + t0 + frow) * a.H + h) * D + fcol;
        if constexpr (!EPI) {
            if (frow < valid) *reinterpret_cast<uint4*>(go) = ov;
        } else {
            float nwv[8], y[8];
            *reinterpret_cast<float4*>(&nwv[0]) = *reinterpret_cast<const float4*>(snw + fcol);
            *reinterpret_cast<float4*>(&nwv[4]) = *reinterpret_cast<const float4*>(snw + fcol + 4);
            gated_rmsnorm_piece<ST, D>(ov, __builtin_bit_cast(uint4, Z), nwv, a.eps, y);
            if (frow < valid) {
                *reinterpret_cast<uint4*>(go) = ov;
                store_vec<ST>(static_cast<ST*>(a.y) + ((size_t)b * a.T + t0 + frow) * a.ld_y + (size_t)h * D + fcol,
                              y);
            }
        }
    };

    // chain waves: fp32 state tiles, rows 16 wr + 4 g4 + e, columns cb + 16 j + r16
    f32x4 S[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
        S[j] = zero4();
        if (chain && a.s0) {
            const float4 x = *reinterpret_cast<const float4*>(a.s0 + ((size_t)bh * D + cb + BS * j + r16) * D +
                                                              BS * wr + 4 * g4);
            S[j] = f32x4{x.x, x.y, x.z, x.w};
        }
    }
    auto put_state = [&]() __attribute__((always_inline)) {   // chain waves: S^T for the B operands
#pragma unroll
        for (int j = 0; j < NTW; ++j)
            *reinterpret_cast<uint2*>(xs + (cb + BS * j + r16) * LDR + BS * wr + 4 * g4) = pack4bf(S[j]);
    };

    // one chunk's A operands, read ahead from its LDS set
    auto preload_kb = [&](const char* sb) __attribute__((always_inline)) {   // chain waves
        const ST* sKb = reinterpret_cast<const ST*>(sb + Lay::KB_OFF);
#pragma unroll
        for (int ks = 0; ks < C / 32; ++ks) Ay[ks] = ldfragT_sw<RB>(sKb, BS * wr, 32 * ks);
        eg = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(sb + Lay::EG_OFF) + BS * wr + 4 * g4);
    };
    auto preload_chain = [&](const char* sb) __attribute__((always_inline)) {
        const ST* sW = reinterpret_cast<const ST*>(sb + Lay::W_OFF);
        const ST* sU = reinterpret_cast<const ST*>(sb + Lay::U_OFF);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) Ax[ks] = ldfrag_sw<RB>(sW, BS * wr, 32 * ks);
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) Rx[j][e] = ld_sw<RB>(sU, BS * wr + 4 * g4 + e, cb + BS * j + r16);
    };
    auto preload_side = [&](const char* sb) __attribute__((always_inline)) {
        const ST* sQp = reinterpret_cast<const ST*>(sb + Lay::QP_OFF);
        const ST* sAqk = reinterpret_cast<const ST*>(sb + Lay::AQK_OFF);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) Ax[ks] = ldfrag_sw<RB>(sQp, BS * wr, 32 * ks);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            if (ks <= wr / 2) Ay[ks] = ldfrag_sw<RB_C>(sAqk, BS * wr, 32 * ks);
    };

    auto chain_step = [&](int n, char* sdma, const char* snext, const char* scur) __attribute__((always_inline)) {
        lds_barrier();                                          // A(n): S^T of chunk n in xs
        Frag8 Bs[NTW][D / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = ldfrag<1, ST>(xs, LDR, cb + BS * j, 32 * ks);
        // V' = U - W S, row block wr, this wave's columns
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            f32x4 P = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) P = mma<1>(Ax[ks], Bs[j][ks], P);
            f32x4 Vp;
#pragma unroll
            for (int e = 0; e < 4; ++e) Vp[e] = Rx[j][e] - P[e];
            *reinterpret_cast<uint2*>(xv + (cb + BS * j + r16) * LDC + BS * wr + 4 * g4) = pack4bf(Vp);
        }
        preload_kb(scur);
        // chunk n+1's slabs landed; chunks up to n+NS-1 may stay in flight
        dma_wait_chunks<L_CHAIN>(min(nc - 1, n + NS - 1) - (n + 1));
        lds_barrier();                                          // B(n): V'^T in xv, chunk n+1 visible
        Frag8 Bv[NTW][C / 32];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bv[j][ks] = ldfrag<1, ST>(xv, LDC, cb + BS * j, 32 * ks);
        // S <- diag(e^G) S + Kb^T V'
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            S[j] = f32x4{S[j][0] * eg.x, S[j][1] * eg.y, S[j][2] * eg.z, S[j][3] * eg.w};
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) S[j] = mma<1>(Ay[ks], Bv[j][ks], S[j]);
        }
        if (n + 1 < nc) put_state();
        // set n % NS is free now (chunk n's operands are all in registers)
        if (n + NS < nc) dma_chunk(n + NS, sdma);
        if (n + 1 < nc) preload_chain(snext);
    };
    auto side_step = [&](int n, const char* snext, const char* scur, f32x4& Zc, const f32x4& Zp)
        __attribute__((always_inline)) {
        lds_barrier();                                          // A(n)
        // O = Qp S + Aqk V', row block wr, columns of half hf: the Qp S half from
        // the chunk-start state in xs before barrier B (beside the chain's V'),
        // the Aqk V' half after it
        f32x4 O[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            O[j] = zero4();
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                O[j] = mma<1>(Ax[ks], ldfrag<1, ST>(xs, LDR, cb + BS * j, 32 * ks), O[j]);
        }
        if (!EPI && n > 0) flush(n - 1, Zp);
        if constexpr (EPI) read_gate(scur, Zc);                 // before B: the set is refilled after it
        lds_barrier();                                          // B(n)
        ST* sst = stg(n);
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (ks <= wr / 2) O[j] = mma<1>(Ay[ks], ldfrag<1, ST>(xv, LDC, cb + BS * j, 32 * ks), O[j]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                st1<ST>(sst + (BS * wr + 4 * g4 + e) * LDU + cb + BS * j + r16, O[j][e]);
        }
        if (EPI && n > 0) flush(n - 1, Zp);
        if (n + 1 < nc) preload_side(snext);
    };

    // Each role runs its own loop (the same barriers in the same order), so no
    // control-flow path joins the two roles' code: a join would make the
    // compiler's wait counts for one role's loads apply to the other's.
    // prologue: chunks 0 .. NS-1 in flight, chunk 0 landed and read
    if (chain) {
        put_state();
        dma_chunk(0, set0);
        if (nc > 1) dma_chunk(1, set1);
        if (NS == 3 && nc > 2) dma_chunk(2, set2);
        dma_wait_chunks<L_CHAIN>(min(NS, nc) - 1);
        lds_barrier();
        preload_chain(set0);
        // unrolled NS times so that every set is named statically
        for (int n = 0; n < nc; n += NS) {
            chain_step(n, set0, set1, set0);
            if (n + 1 < nc) chain_step(n + 1, set1, NS == 3 ? set2 : set0, set1);
            if (NS == 3 && n + 2 < nc) chain_step(n + 2, set2, set0, set2);
        }
        lds_barrier();
        if (a.s_final) {
#pragma unroll
            for (int j = 0; j < NTW; ++j)
                *reinterpret_cast<float4*>(a.s_final + ((size_t)bh * D + cb + BS * j + r16) * D + BS * wr + 4 * g4) =
                    make_float4(S[j][0], S[j][1], S[j][2], S[j][3]);
        }
    } else {
        lds_barrier();
        preload_side(set0);
        static_assert(!EPI || NS == 2, "gate register sets alternate with the LDS sets");
        for (int n = 0; n < nc; n += NS) {
            side_step(n, set1, set0, Rx[0], Rz[0]);
            if (n + 1 < nc) side_step(n + 1, NS == 3 ? set2 : set0, set1, Rz[0], Rx[0]);
            if (NS == 3 && n + 2 < nc) side_step(n + 2, set0, set2, Rx[0], Rz[0]);
        }
        lds_barrier();
        if ((nc - 1) & 1)   // a static pick of the register set (a selected array would live in scratch)
            flush(nc - 1, Rz[0]);
        else
            flush(nc - 1, Rx[0]);
    }
}

template <int D, int CS>
struct Dh3Layout {
    static constexpr int DC = D / CS, NS = 3;
    static constexpr int RB_D = 2 * D, RB_C = 2 * C, RB_U = 2 * DC;
    // Aqk, Qp and W are read transposed (Aqk^T, Qp^T, W^T) with transposing LDS reads
    static constexpr int AQK_OFF = 0;                                         // [C][C]
    static constexpr int KB_OFF = AQK_OFF + C * RB_C;                         // [C][D]
    static constexpr int QP_OFF = KB_OFF + C * RB_D;                          // [C][D]
    static constexpr int W_OFF = QP_OFF + C * RB_D;                           // [C][D]
    static constexpr int DO_OFF = W_OFF + C * RB_D;                           // [C][DC] (t, own columns)
    static constexpr int EG_OFF = DO_OFF + C * RB_U;                          // [D] fp32
    static constexpr int SET_BYTES = (EG_OFF + 4 * D + 1023) & ~1023;
    // Staging rows (LDU) keep a 16-byte pad for 16-byte row access.  The
    // exchange tiles (LDR, LDC) are only touched 8 bytes at a time: a 4-element
    // pad (rows of 34 dwords, 2 mod 32) puts the 16 rows of a fragment read or
    // a C-layout write in 16 distinct bank pairs.
    static constexpr int PS = 8, PX = 4, LDR = D + PX, LDU = DC + PS, LDC = C + PX;
    static constexpr int XS_OFF = 0;                                          // dS^T   [DC][LDR]
    static constexpr int XV_OFF = XS_OFF + DC * LDR * 2;                      // -dV'^T [DC][LDC]
    static constexpr int STG_OFF = XV_OFF + DC * LDC * 2;
    static constexpr int STG_ELEMS = D * LDU + C * LDU;                       // dh, dV'
    static constexpr int STG_BYTES = (STG_ELEMS * 2 + 15) & ~15;
    static constexpr int NSTG = 3;
    static constexpr int XBYTES = STG_OFF + NSTG * STG_BYTES;
    static_assert(NS * SET_BYTES + XBYTES <= 160 * 1024, "reverse recurrence LDS");
    static constexpr int L =
        DmaTile<C, RB_C, 4>::COUNT + 3 * DmaTile<C, RB_D, 4>::COUNT + DmaTile<C, RB_U, 4>::COUNT + 1;
};

// ----------------------------------------------------------------------------
// kda_dh4_kernel: the reverse state recurrence (loop step k on chunk
// nc-1-k), the pipeline of kda_recur3_kernel with the work split between
// two wave roles (512 threads).  Waves 0-3 run the reverse state chain: dV' (row block wr),
// the dS update of state rows wr, wr + 4, the dS^T and -dV'^T exchange tiles,
// and read the next chunk's operands (dO^T by transposing reads of the set's
// dO tile).  Waves 4-7 bring the slabs by DMA (after barrier B, when the
// step's set is free) and copy the step's outputs straight from the exchange
// tiles: dh from dS^T before barrier B, dV' from -dV'^T after it.
// ----------------------------------------------------------------------------
template <int D, int CS>
struct Dh4Layout {
    using B3 = Dh3Layout<D, CS>;
    static constexpr int DC = B3::DC, NS = B3::NS, SET_BYTES = B3::SET_BYTES;
    static constexpr int LDR = B3::LDR, LDU = B3::LDU, LDC = B3::LDC;
    static constexpr int XS_OFF = B3::XS_OFF, XV_OFF = B3::XV_OFF;
    static constexpr int XBYTES = B3::STG_OFF;                                 // the two exchange tiles
    static_assert(NS * SET_BYTES + XBYTES <= 160 * 1024, "reverse recurrence LDS");
};

template <int D, int CS>
__global__ __launch_bounds__(512) void kda_dh4_kernel(const DhArgs a) {
    using ST = uint16_t;
    using B3 = Dh3Layout<D, CS>;
    using Lay = Dh4Layout<D, CS>;
    constexpr int NT = D / BS, DC = Lay::DC, NTW = DC / BS, MT = (NT + 3) / 4, NS = Lay::NS;
    constexpr int LDR = Lay::LDR, LDC = Lay::LDC;
    constexpr int RB_D = B3::RB_D, RB_C = B3::RB_C, RB_U = B3::RB_U;
    static_assert(NS == 3, "three DMA sets");
    __shared__ __align__(1024) char set0[Lay::SET_BYTES];
    __shared__ __align__(1024) char set1[Lay::SET_BYTES];
    __shared__ __align__(1024) char set2[Lay::SET_BYTES];
    __shared__ __align__(16) char smem[Lay::XBYTES];

    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, r16 = l & 15, g4 = l >> 4;
    __builtin_assume(w >= 0 && w < 8);
    const int role = w >> 2, wr = w & 3;
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lb / CS, c0 = (lb - bh * CS) * DC;
    const int b = bh / a.H, h = bh - b * a.H;
    const int nc = a.nc;
    const char* gAqk = static_cast<const char*>(a.Aqk);
    const char* gKb = static_cast<const char*>(a.Kb);
    const char* gQp = static_cast<const char*>(a.Qp);
    const char* gW = static_cast<const char*>(a.W);
    const char* gdO = static_cast<const char*>(a.dout);
    const char* gEg = reinterpret_cast<const char*>(a.eG);

    ST* xs = reinterpret_cast<ST*>(smem + Lay::XS_OFF);
    ST* xv = reinterpret_cast<ST*>(smem + Lay::XV_OFF);

    // step k's slabs (chunk nc-1-k) -> LDS set (k % NS), by the role-1 waves
    using TA = DmaTile<C, RB_C, 4>;   // Aqk
    using TB = DmaTile<C, RB_D, 4>;   // Kb, Qp, W
    using TO = DmaTile<C, RB_U, 4>;
    constexpr int L = B3::L;
    uint32_t oA[TA::COUNT], oB[TB::COUNT], oO[TO::COUNT];
    TA::offsets(oA, RB_C, wr, l);
    TB::offsets(oB, RB_D, wr, l);
    TO::offsets(oO, (size_t)a.H * D * 2, wr, l);
    const uint32_t oE = (uint32_t)((D / 4) * 4 * wr + 16 * (l < D / 16 ? l : 0));
    auto dma_step = [&](int k, char* sbp) __attribute__((always_inline)) {
        const int n = nc - 1 - k;
        const size_t ch = (size_t)bh * nc + n;
        const int t0 = n * C, valid = min(C, a.T - t0);
        const uint32_t sb = lds_addr(sbp);
        TA::issue_s32(gAqk + ch * C * C * 2, oA, sb + B3::AQK_OFF, wr);
        TB::issue_s32(gKb + ch * C * D * 2, oB, sb + B3::KB_OFF, wr);
        TB::issue_s32(gQp + ch * C * D * 2, oB, sb + B3::QP_OFF, wr);
        TB::issue_s32(gW + ch * C * D * 2, oB, sb + B3::W_OFF, wr);
        const char* gdo = gdO + ((((size_t)b * a.T + t0) * a.H + h) * D + c0) * 2;
        if (valid == C) TO::issue_s32(gdo, oO, sb + B3::DO_OFF, wr);
        else TO::issue(gdo, (size_t)a.H * D * 2, sbp + B3::DO_OFF, wr, l, valid);
        if (l < D / 16) dma16_s32(gEg + ch * D * 4, oE, sb + B3::EG_OFF + D * wr);
    };
    // The rows of the partial chunk's dO tile past T (not loaded by the DMA) are
    // cleared once, by the role-1 waves, so that its dO^T fragments read zeros
    // there: 16 bytes per thread, whole rows, so the swizzle does not matter.
    auto clear_do_tail = [&](char* sb) __attribute__((always_inline)) {
        static_assert(C * RB_U == 256 * 16, "one 16-byte piece per role-1 thread");
        const int t1 = tid - 256, row = t1 / (RB_U / 16);
        const int valid = a.T - (nc - 1) * C;
        if (row >= valid) *reinterpret_cast<uint4*>(sb + B3::DO_OFF + 16 * t1) = make_uint4(0u, 0u, 0u, 0u);
    };
    // Outputs of step k, by the role-1 waves from the exchange tiles, as 16-byte
    // row pieces by transposing reads (one piece per thread and tile): dh from
    // dS^T in xs (there between A(k) and B(k)), dV' from -dV'^T in xv (there
    // between B(k) and A(k+1)), negated back
    static_assert(DC == 32 && D * DC / 8 == 256 && C * DC / 8 == 256, "one 16-byte piece per role-1 thread");
    const int t1 = tid - 256, pi = t1 & 15, prow = 4 * (t1 >> 4) + (pi & 3), pcol = c0 + 8 * (pi >> 2);
    auto copy_dh = [&](int k) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * nc + (nc - 1 - k);
        const short8v x = ld_tr_rows8(xs, LDR, 0, 4 * (t1 >> 4));
        *reinterpret_cast<short8v*>(static_cast<ST*>(a.dh) + ch * D * D + (size_t)prow * D + pcol) = x;
    };
    auto copy_dvp = [&](int k) __attribute__((always_inline)) {
        const size_t ch = (size_t)bh * nc + (nc - 1 - k);
        const short8v x = ld_tr_rows8(xv, LDC, 0, 4 * (t1 >> 4)) ^ short8v{(short)0x8000, (short)0x8000,
            (short)0x8000, (short)0x8000, (short)0x8000, (short)0x8000, (short)0x8000, (short)0x8000};
        *reinterpret_cast<short8v*>(static_cast<ST*>(a.dVp) + ch * C * D + (size_t)prow * D + pcol) = x;
    };

    int mt[MT];
    bool own[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        mt[i] = wr + 4 * i;
        own[i] = role == 0 && mt[i] < NT;
    }
    f32x4 dS[MT][NTW];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            dS[i][j] = zero4();
            if (own[i] && a.dsf) {
                const float4 x = *reinterpret_cast<const float4*>(
                    a.dsf + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4);
                dS[i][j] = f32x4{x.x, x.y, x.z, x.w};
            }
        }
    auto put_state = [&]() __attribute__((always_inline)) {   // chain waves
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<uint2*>(xs + (BS * j + r16) * LDR + BS * mt[i] + 4 * g4) = pack4bf(dS[i][j]);
    };

    Frag8 Aat[2], Akb[D / 32], Aqt[MT][C / 32], Awt[MT][C / 32], Bo[NTW][C / 32];
    f32x4 dVa[NTW];   // the chunk's A_qk^T dO part of dV', formed with its operands
    float4 eg[MT];
    auto preload = [&](const char* sb) __attribute__((always_inline)) {   // chain waves
        const ST* sAqk = reinterpret_cast<const ST*>(sb + B3::AQK_OFF);
        const ST* sKb = reinterpret_cast<const ST*>(sb + B3::KB_OFF);
        const ST* sQp = reinterpret_cast<const ST*>(sb + B3::QP_OFF);
        const ST* sW = reinterpret_cast<const ST*>(sb + B3::W_OFF);
        const float* seG = reinterpret_cast<const float*>(sb + B3::EG_OFF);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            if (ks >= wr / 2) Aat[ks] = ldfragT_sw<RB_C>(sAqk, BS * wr, 32 * ks);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) Akb[ks] = ldfrag_sw<RB_D>(sKb, BS * wr, 32 * ks);
        const ST* sdO = reinterpret_cast<const ST*>(sb + B3::DO_OFF);
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int ks = 0; ks < C / 32; ++ks) Bo[j][ks] = ldfragT_sw<RB_U>(sdO, BS * j, 32 * ks);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i]) {
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) {
                    Aqt[i][ks] = ldfragT_sw<RB_D>(sQp, BS * mt[i], 32 * ks);
                    Awt[i][ks] = ldfragT_sw<RB_D>(sW, BS * mt[i], 32 * ks);
                }
                eg[i] = *reinterpret_cast<const float4*>(seG + BS * mt[i] + 4 * g4);
            }
        // A_qk^T dO does not depend on the chain: formed here, off barrier A's path
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            dVa[j] = zero4();
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (ks >= wr / 2) dVa[j] = mma<1>(Aat[ks], Bo[j][ks], dVa[j]);
        }
    };

    // prologue: steps 0 .. NS-1 in flight; step 0's operands read
    if (role == 0) put_state();
    if (role == 1) {
        dma_step(0, set0);
        if (nc > 1) dma_step(1, set1);
        if (nc > 2) dma_step(2, set2);
        dma_wait_chunks<L>(min(NS, nc) - 1);
        if (a.T < nc * C) clear_do_tail(set0);
    }
    lds_barrier();
    if (role == 0) preload(set0);

    // step k: chunk nc-1-k in set k % NS
    auto step = [&](int k, char* scur, const char* snext) __attribute__((always_inline)) {
        lds_barrier();                                          // A(k): dS^T in xs
        if (role == 0) {
            Frag8 Bs[NTW][D / 32];
#pragma unroll
            for (int j = 0; j < NTW; ++j)
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) Bs[j][ks] = ldfrag<1, ST>(xs, LDR, BS * j, 32 * ks);
            // dV' = Aqk^T dO + Kb dS, row block wr
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                f32x4 dV = dVa[j];
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) dV = mma<1>(Akb[ks], Bs[j][ks], dV);
                *reinterpret_cast<uint2*>(xv + (BS * j + r16) * LDC + BS * wr + 4 * g4) = pack4bf(negacc(dV));
            }
        } else {
            // step k+1's slabs landed (chunks up to k+NS-1 may stay in flight)
            if (k + 1 < nc) dma_wait_chunks<L>(min(nc - 1, k + NS - 1) - (k + 1));
            copy_dh(k);   // after the wait: a store issued before it would hold the count
        }
        lds_barrier();                                          // B(k): -dV'^T in xv, step k+1's slabs
        if (role == 0) {
            Frag8 Bvn[NTW][C / 32];    // -dV'
#pragma unroll
            for (int j = 0; j < NTW; ++j)
#pragma unroll
                for (int ks = 0; ks < C / 32; ++ks) Bvn[j][ks] = ldfrag<1, ST>(xv, LDC, BS * j, 32 * ks);
            // dS <- diag(e^G) dS + Qp^T dO - W^T dV'
#pragma unroll
            for (int i = 0; i < MT; ++i)
                if (own[i]) {
#pragma unroll
                    for (int j = 0; j < NTW; ++j) {
                        dS[i][j] = f32x4{dS[i][j][0] * eg[i].x, dS[i][j][1] * eg[i].y, dS[i][j][2] * eg[i].z,
                                         dS[i][j][3] * eg[i].w};
#pragma unroll
                        for (int ks = 0; ks < C / 32; ++ks) {
                            dS[i][j] = mma<1>(Awt[i][ks], Bvn[j][ks], dS[i][j]);
                            dS[i][j] = mma<1>(Aqt[i][ks], Bo[j][ks], dS[i][j]);
                        }
                    }
                }
            if (k + 1 < nc) {
                put_state();
                preload(snext);
            }
        } else {
            // set k % NS is free: chunk k's operands, dO^T included, are in the
            // chain waves' registers
            if (k + NS < nc) dma_step(k + NS, scur);
            copy_dvp(k);
        }
    };
    for (int k = 0; k < nc; k += 3) {
        step(k, set0, set1);
        if (k + 1 < nc) step(k + 1, set1, set2);
        if (k + 2 < nc) step(k + 2, set2, set0);
    }

    if (a.ds0) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (own[i])
#pragma unroll
                for (int j = 0; j < NTW; ++j)
                    *reinterpret_cast<float4*>(a.ds0 + ((size_t)bh * D + c0 + BS * j + r16) * D + BS * mt[i] + 4 * g4) =
                        make_float4(dS[i][j][0], dS[i][j][1], dS[i][j][2], dS[i][j][3]);
    }
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
// D = 128 splits the state's dv columns over two workgroups per (batch, head)
// bf16: row-split kernels with CS2 workgroups per (batch, head); fp32: one
// workgroup per (batch, head), D = 128 split over two.
template <int D> struct RowSplit { static constexpr int CS = (D >= 128) ? 4 : 2; };

template <int D, typename ST, int MODE>
static hipError_t launch_recur_t(const RecurArgs& a, hipStream_t st) {
    if (a.y != nullptr) {
        // the forward with the gated RMSNorm fused into the O store: kernels whose
        // workgroup holds whole output rows
        if constexpr (MODE == 0 && std::is_same<ST, uint16_t>::value && D == 64)
            hipLaunchKernelGGL((kda_recur5_kernel<D, true>), dim3(a.BH), dim3(1024), 0, st, a);
        else if constexpr (MODE == 0 && std::is_same<ST, float>::value && D <= 64)
            hipLaunchKernelGGL((kda_recur_kernel<D, ST, 3, 0, 1, true>), dim3(a.BH), dim3(256), 0, st, a);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if constexpr (std::is_same<ST, uint16_t>::value && D == 64) {
        if (a.Kb == nullptr) return hipErrorInvalidValue;
        constexpr int CS2 = RowSplit<D>::CS;
        hipLaunchKernelGGL((kda_recur4_kernel<D, MODE, CS2>), dim3(a.BH * CS2), dim3(512), 0, st, a);
    } else if constexpr (std::is_same<ST, uint16_t>::value && D >= 64) {
        constexpr int CS2 = RowSplit<D>::CS;
        hipLaunchKernelGGL((kda_recur3_kernel<D, MODE, CS2>), dim3(a.BH * CS2), dim3(256), 0, st, a);
    } else if constexpr (std::is_same<ST, uint16_t>::value) {
        constexpr int CS2 = RowSplit<D>::CS;
        hipLaunchKernelGGL((kda_recur2_kernel<D, MODE, CS2>), dim3(a.BH * CS2), dim3(512), 0, st, a);
    } else {
        constexpr int CS = (D >= 128) ? 2 : 1;
        hipLaunchKernelGGL((kda_recur_kernel<D, ST, 3, MODE, CS>), dim3(a.BH * CS), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <int D, typename ST>
static hipError_t launch_dh_t(const DhArgs& a, hipStream_t st) {
    if constexpr (std::is_same<ST, uint16_t>::value && D >= 64) {
        if (!a.Aqk || !a.Qp || !a.W || !a.Kb) return hipErrorInvalidValue;
        constexpr int CS2 = RowSplit<D>::CS;
        hipLaunchKernelGGL((kda_dh4_kernel<D, CS2>), dim3(a.BH * CS2), dim3(512), 0, st, a);
    } else if constexpr (std::is_same<ST, uint16_t>::value) {
        constexpr int CS2 = RowSplit<D>::CS;
        hipLaunchKernelGGL((kda_dh2_kernel<D, CS2>), dim3(a.BH * CS2), dim3(512), 0, st, a);
    } else {
        hipLaunchKernelGGL((kda_dh_kernel<D, ST, 3>), dim3(a.BH), dim3(256), 0, st, a);
    }
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
    if (D == 128 && mode == 0)
        return in_bf16 ? launch_recur_t<128, uint16_t, 0>(a, st) : launch_recur_t<128, float, 0>(a, st);
    // the backward's state recompute at D = 128: the generic kernel, which also
    // writes V' for the D = 128 local-adjoint kernel; two workgroups per
    // (batch, head), 64 dv columns each
    if (D == 128 && mode == 1) {
        if (a.Vp == nullptr || a.KbT == nullptr) return hipErrorInvalidValue;
        if (in_bf16)
            hipLaunchKernelGGL((kda_recur_kernel<128, uint16_t, 1, 1, 2>), dim3(a.BH * 2), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((kda_recur_kernel<128, float, 3, 1, 2>), dim3(a.BH * 2), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

bool recur_epilogue_supported(int D, int in_bf16) { return in_bf16 ? D == 64 : (D == 32 || D == 64); }

// The reverse carry over segments (bf16, D = 128): the segments' reverse maps
// X_rev (a.segX), the reverse scan (a.segS, launched by the caller between the
// two), then every segment's dh, dV' and dS0.
hipError_t launch_dh_seg_maps(const DhArgs& a, hipStream_t st) {
    if (a.nseg < 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL((kda_dh_kernel<128, uint16_t, 1, 2, 1>), dim3(a.BH * 2 * (a.nseg - 1)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_dh_seg(const DhArgs& a, hipStream_t st) {
    if (a.nseg < 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL((kda_dh_kernel<128, uint16_t, 1, 2, 2>), dim3(a.BH * 2 * a.nseg), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_states_dh(const RecurArgs& ra, const DhArgs& da, hipStream_t st) {
    if (ra.BH != da.BH || !ra.Vp || !ra.KbT || !da.AqkT || !da.QpT || !da.WT || !da.Kb) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kda_states_dh_kernel, dim3(4 * ra.BH), dim3(256), 0, st, ra, da);
    return hipGetLastError();
}

hipError_t launch_dh(const DhArgs& a, int D, int in_bf16, hipStream_t st) {
    if (D == 32) return in_bf16 ? launch_dh_t<32, uint16_t>(a, st) : launch_dh_t<32, float>(a, st);
    if (D == 64) return in_bf16 ? launch_dh_t<64, uint16_t>(a, st) : launch_dh_t<64, float>(a, st);
    // D = 128: the generic kernel on the transposed slabs; bf16: two workgroups
    // per (batch, head), 64 dS columns each (one column tile per wave); fp32:
    // four, 32 dS columns each (one operand set and its staging fit the LDS
    // only at that width)
    if (D == 128) {
        if (!a.AqkT || !a.QpT || !a.WT || !a.Kb) return hipErrorInvalidValue;
        if (in_bf16)
            hipLaunchKernelGGL((kda_dh_kernel<128, uint16_t, 1, 2>), dim3(a.BH * 2), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((kda_dh_kernel<128, float, 3, 4>), dim3(a.BH * 4), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

}  // namespace kda
