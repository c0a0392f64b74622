// kda_api.hip -- the C ABI declared in include/kda_hip.h: argument checks,
// workspace layout and the launch sequence of the forward and backward passes.
// Also the standalone unit-triangular solve and a small state-copy kernel.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "kda_hip.h"
#include "kda_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return KDA_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

struct Layout {
    int64_t off[KDA_WS_NREGIONS];
    size_t total;
    // pass 2: bytes of the regions the training forward writes and the
    // backward reads (placed first); the backward's own regions follow.
    // Passes 0 and 1: total.
    size_t kept;
    // pass 2, a forward over segments: its segment temporaries (X, M, S, segf_per
    // bytes each from segf), unnamed bytes at the end of the kept part that only
    // the training forward writes; -1: none
    int64_t segf = -1;
    size_t segf_per = 0;
};

// regions only the backward writes and reads (the training pair's scratch)
bool backward_region(int r) {
    return r == KDA_WS_H || r == KDA_WS_DH || r == KDA_WS_VP || r == KDA_WS_DVP || r == KDA_WS_PADB ||
           r == KDA_WS_SEGX || r == KDA_WS_SEGM || r == KDA_WS_SEGS;
}

int check_shape(int B, int T, int H, int D, int chunk, int dtype, int g_dtype, bool bwd) {
    if (B < 0 || T < 0 || H < 0) return fail(KDA_E_INVALID, "negative size: B=%d T=%d H=%d", B, T, H);
    // the reference's chunk sizes; the kernels block at kda::C whatever the value
    // (the chunked recurrence's result does not depend on the chunk size)
    if (chunk != 8 && chunk != 16 && chunk != 32 && chunk != kda::C)
        return fail(KDA_E_UNSUPPORTED, "chunk=%d: expected 8, 16, 32 or 64", chunk);
    if (D != 32 && D != 64 && D != 96 && D != 128)
        return fail(KDA_E_UNSUPPORTED, "D=%d: the %s supports D in {32, 64, 96, 128}", D,
                    bwd ? "backward" : "forward");
    if (dtype != KDA_DTYPE_F32 && dtype != KDA_DTYPE_BF16)
        return fail(KDA_E_UNSUPPORTED, "dtype=%d: expected 0 (fp32) or 1 (bf16)", dtype);
    if (g_dtype != KDA_DTYPE_F32 && g_dtype != KDA_DTYPE_BF16 && g_dtype != KDA_G_HEAD_F32)
        return fail(KDA_E_UNSUPPORTED, "g_dtype=%d: expected 0 (fp32), 1 (bf16) or 2 (fp32, one per head)",
                    g_dtype);
    if (g_dtype == KDA_G_HEAD_F32 && (dtype != KDA_DTYPE_BF16 || (D != 32 && D != 64)))
        return fail(KDA_E_UNSUPPORTED, "g_dtype=2 (one decay per head) needs bf16 operands and D in {32, 64}; "
                    "got dtype=%d D=%d (broadcast g over the channels instead)", dtype, D);
    const long long nchunks = (long long)B * H * ((T + kda::C - 1) / kda::C);
    if (nchunks > 0x7fffffffLL) return fail(KDA_E_UNSUPPORTED, "B*H*ceil(T/64)=%lld exceeds 2^31-1", nchunks);
    return KDA_OK;
}

// Whether the forward runs segmented (kda_seg.hip): bf16 at D = 128 when the
// plan has at least 8 segments or segments of at least 32 chunks.  A chunk of
// a segment costs the two segment passes about 3.5 times a chunk of the
// one-chain-per-(b, h) forward, so short segments lose: at B8 H8 T1568 (4
// segments of 7 chunks) the forward took 181 us segmented against 153 us
// unsegmented; with 4 segments of 16 chunks or 2 of 13 the two were level.
// Passes 0 and 2 (the training forward).  *nseg / *seg_len: the plan.
bool seg_forward(int pass, int B, int T, int H, int D, int dtype, int* nseg, int* seg_len) {
    *nseg = 1;
    *seg_len = 0;
    if (pass == KDA_PASS_BWD || dtype != KDA_DTYPE_BF16 || D != 128 || (size_t)B * T * H == 0) return false;
    kda::seg_plan(B * H, (T + kda::C - 1) / kda::C, nseg, seg_len);
    if (*nseg > 1 && (*nseg >= 8 || *seg_len >= 32)) return true;
    *nseg = 1;
    *seg_len = 0;
    return false;
}

// Whether the backward's state recompute and reverse carry run segmented (the
// same plan; passes A and B, then the chunk-start states per segment; the
// segments' reverse maps, a reverse scan and the segments' dh): bf16 at the
// kernels' D = 128 when the plan has at least SEG_STATES_MIN segments.  The
// segment passes read the chunk slabs twice (maps, then states), about 1.4x
// the bytes of one chain per (b, h), and take about 3.4 times as long per
// chunk of a segment as that chain per chunk at D = 128 (SSv2's shape, 64
// (b, h) x 25 chunks, 4 segments: 95 against 87 us); with 8 or more segments
// (at most 32 (b, h)) the segments' length, not the sequence's, sets the time.
constexpr int SEG_STATES_MIN = 8;
bool seg_states(int pass, int B, int T, int H, int D, int dtype, int* nseg, int* seg_len) {
    *nseg = 1;
    *seg_len = 0;
    if (pass == KDA_PASS_FWD || dtype != KDA_DTYPE_BF16 || D != 128 || (size_t)B * T * H == 0) return false;
    kda::seg_plan(B * H, (T + kda::C - 1) / kda::C, nseg, seg_len);
    if (*nseg >= SEG_STATES_MIN) return true;
    *nseg = 1;
    *seg_len = 0;
    return false;
}

// D = 96 runs the D = 128 kernels.  The prep and the local-adjoint kernel read
// q, k, v, g (and dout) rows of 96 channels themselves, the missing channels
// as zero, and write dq, dk, dv, dg rows of 96; o, dout for the reverse carry
// and the states go through zero-padded copies (kda_pad.hip) in the PAD and
// PADB regions, in these slots.
constexpr int PAD_D = 128;
bool padded_head(int D) { return D == 96; }
enum PadSlot { PS_O, PS_DO, PS_S0, PS_SF, PS_DSF, PS_DS0, PS_N };

// The slots of the backward's padded cotangents and gradients live in the
// PADB region, the others (the initial state, the forward's outputs) in PAD.
bool pad_backward_slot(int i) { return i == PS_DO || i == PS_DSF || i == PS_DS0; }

struct PadLayout {
    size_t off[PS_N];   // within the slot's region
    size_t total;       // PAD
    size_t total_b;     // PADB
};

void make_pad_layout(int pass, int B, int T, int H, int dtype, PadLayout& P) {
    const size_t tok = (size_t)B * T * H * PAD_D, es = (dtype == KDA_DTYPE_BF16) ? 2 : 4;
    const size_t st = (size_t)B * H * PAD_D * PAD_D * 4;
    size_t sz[PS_N] = {0};
    sz[PS_S0] = st;
    if (pass != KDA_PASS_BWD) {
        sz[PS_O] = tok * es;
        sz[PS_SF] = st;
    }
    if (pass != KDA_PASS_FWD) {
        sz[PS_DO] = tok * es;
        sz[PS_DSF] = sz[PS_DS0] = st;
    }
    size_t cur = 0, curb = 0;
    for (int i = 0; i < PS_N; ++i) {
        size_t& c = pad_backward_slot(i) ? curb : cur;
        P.off[i] = c;
        c += (sz[i] + 255) & ~(size_t)255;
    }
    P.total = cur;
    P.total_b = curb;
}

// Region sizes in bytes at the kernels' head dimension D.  Operand slabs use
// the input dtype's element size; eG, Akk and Tii are fp32.  Akk, Tii and V'
// exist for fp32 inputs and at D = 128 only.
void region_sizes(int pass, int B, int T, int H, int D, int dtype, size_t* sz) {
    const size_t nc = (size_t)(T + kda::C - 1) / kda::C;
    const size_t N = (size_t)B * H * nc;
    const size_t es = (dtype == KDA_DTYPE_BF16) ? 2 : 4;
    const size_t CD = N * kda::C * D * es, CC = N * kda::C * kda::C * es, DD = N * (size_t)D * D * es;
    const size_t TI = N * kda::NB * kda::BS * kda::BS * 4, EG = N * D * 4;
    // bf16 D = 64: the recurrences read Kb, Qp, W and Aqk through transposing LDS
    // reads, so no transposed slab exists and both passes use Qp and Aqk
    const bool tr = dtype == KDA_DTYPE_BF16 && D == 64;
    sz[KDA_WS_W] = CD;
    sz[KDA_WS_U] = CD;
    sz[KDA_WS_KBT] = tr ? 0 : CD;
    sz[KDA_WS_KB] = tr ? CD : 0;
    sz[KDA_WS_EG] = EG;
    if (pass != KDA_PASS_BWD || tr) {
        sz[KDA_WS_QP] = CD;
        sz[KDA_WS_AQK] = CC;
    }
    if (pass != KDA_PASS_FWD) {
        sz[KDA_WS_WT] = tr ? 0 : CD;
        sz[KDA_WS_QPT] = tr ? 0 : CD;
        sz[KDA_WS_KB] = CD;
        sz[KDA_WS_AQKT] = tr ? 0 : CC;
        sz[KDA_WS_H] = DD;
        sz[KDA_WS_DH] = DD;
        sz[KDA_WS_DVP] = CD;
        if (dtype == KDA_DTYPE_F32 || D == 128) {
            // the bf16 local-adjoint kernel at D <= 64 recomputes these from the
            // chunk's inputs; the fp32 one and the one at D = 128 read them
            sz[KDA_WS_AKK] = N * kda::C * kda::C * 4;
            sz[KDA_WS_TII] = TI;
            sz[KDA_WS_VP] = CD;
        }
    }
    // the named segment regions: the forward's (pass 0) and the backward's;
    // the training forward's temporaries are unnamed (make_layout)
    int nseg, seg_len;
    if ((pass == KDA_PASS_FWD && seg_forward(pass, B, T, H, D, dtype, &nseg, &seg_len)) ||
        seg_states(pass, B, T, H, D, dtype, &nseg, &seg_len)) {
        const size_t per = (size_t)B * H * nseg * D * D * 4;
        sz[KDA_WS_SEGX] = per;
        sz[KDA_WS_SEGM] = per;
        sz[KDA_WS_SEGS] = per;
    }
}

// Passes 0 and 1: the regions in enum order.  Pass 2: the regions the
// training forward writes first, then the backward's own.  D = 96: the D = 128
// regions and the PAD / PADB regions of the padded copies.
void make_layout(int pass, int B, int T, int H, int D, int dtype, Layout& L) {
    size_t sz[KDA_WS_NREGIONS] = {0};
    region_sizes(pass, B, T, H, padded_head(D) ? PAD_D : D, dtype, sz);
    if (padded_head(D)) {
        PadLayout P;
        make_pad_layout(pass, B, T, H, dtype, P);
        sz[KDA_WS_PAD] = P.total;
        sz[KDA_WS_PADB] = P.total_b;
    }
    size_t cur = 0;
    auto place = [&](int r) {
        if (sz[r] == 0) {
            L.off[r] = -1;
            return;
        }
        L.off[r] = (int64_t)cur;
        cur += (sz[r] + 255) & ~(size_t)255;
    };
    if (pass == KDA_PASS_TRAIN) {
        for (int r = 0; r < KDA_WS_NREGIONS; ++r)
            if (!backward_region(r)) place(r);
        // the training forward over segments: its temporaries, in the kept part
        // (the forward is given only that part; the backward does not touch them)
        int nseg, seg_len;
        const int Dk = padded_head(D) ? PAD_D : D;
        if (seg_forward(pass, B, T, H, Dk, dtype, &nseg, &seg_len)) {
            L.segf_per = ((size_t)B * H * nseg * Dk * Dk * 4 + 255) & ~(size_t)255;
            L.segf = (int64_t)cur;
            cur += 3 * L.segf_per;
        }
        L.kept = cur;
        for (int r = 0; r < KDA_WS_NREGIONS; ++r)
            if (backward_region(r)) place(r);
    } else {
        for (int r = 0; r < KDA_WS_NREGIONS; ++r) place(r);
        L.kept = cur;
    }
    L.total = cur;
}

// The regions' addresses: those below L.kept in `kept`, the others in
// `scratch` (null: the caller touches none of them).
struct Ws {
    void* r[KDA_WS_NREGIONS];
    char* segf;        // the training forward's segment temporaries (X, M, S), or null
    size_t segf_per;
};

Ws resolve(const Layout& L, void* kept, void* scratch) {
    Ws w;
    w.segf = L.segf >= 0 ? static_cast<char*>(kept) + L.segf : nullptr;
    w.segf_per = L.segf_per;
    for (int r = 0; r < KDA_WS_NREGIONS; ++r) {
        const int64_t o = L.off[r];
        if (o < 0)
            w.r[r] = nullptr;
        else if ((size_t)o < L.kept)
            w.r[r] = static_cast<char*>(kept) + o;
        else
            w.r[r] = scratch ? static_cast<char*>(scratch) + (o - (int64_t)L.kept) : nullptr;
    }
    return w;
}

void* region(const Ws& ws, int r) { return ws.r[r]; }
float* fregion(const Ws& ws, int r) { return static_cast<float*>(ws.r[r]); }

int check_io(const void* p, const char* name, int /*dtype*/, bool nullable) {
    if (!p) return nullable ? KDA_OK : fail(KDA_E_INVALID, "%s is NULL", name);
    if (!aligned(p, 16)) return fail(KDA_E_INVALID, "%s is not 16-byte aligned", name);
    return KDA_OK;
}

int check_scalar(const void* p, const char* name, int dtype) {
    if (!p) return fail(KDA_E_INVALID, "%s is NULL", name);
    if (!aligned(p, dtype == KDA_DTYPE_F32 ? 4 : 2)) return fail(KDA_E_INVALID, "%s is misaligned", name);
    return KDA_OK;
}

int hip_fail(hipError_t e, const char* where) {
    return fail(KDA_E_HIP, "%s: %s", where, hipGetErrorString(e));
}

// ---- optional launch timing: an event pair around each launch, on its stream ----
enum { PROF_PREP_FWD = 0, PROF_RECUR_FWD, PROF_PREP_BWD, PROF_RECUR_H, PROF_DH, PROF_LOCAL, PROF_PREP_TRAIN,
       PROF_PRODUCER_FWD, PROF_PRODUCER_BWD, PROF_RMSNORM_FWD, PROF_RMSNORM_BWD, PROF_SEG_MAP, PROF_SEG_SCAN,
       PROF_SEG_FWD, PROF_STATES_DH };
const char* const kProfNames[KDA_PROF_NKERNELS] = {"kda_prep_kernel(fwd)", "kda_recur_kernel(fwd)",
                                                   "kda_prep_kernel(bwd)", "kda_recur_kernel(states)",
                                                   "kda_dh_kernel", "kda_bwd_local_kernel",
                                                   "kda_prep_kernel(train)", "producer_fwd_kernel",
                                                   "producer_bwd_kernel(+reduce)", "rmsnorm_fwd_kernel",
                                                   "rmsnorm_bwd_kernel(+reduce)", "kda_segchain_kernel(map)",
                                                   "kda_segscan_kernel", "kda_segchain_kernel(fwd)",
                                                   "kda_states_dh_kernel(states + dh)"};
struct Profiler {
    std::mutex mu;
    bool on = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pool[KDA_PROF_NKERNELS];
    size_t used[KDA_PROF_NKERNELS] = {};
};
Profiler& profiler() {
    static Profiler p;
    return p;
}
int prof_start(int id, hipStream_t st) {
    Profiler& P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    if (!P.on) return -1;
    if (P.used[id] == P.pool[id].size()) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess) return -1;
        if (hipEventCreate(&b) != hipSuccess) {
            (void)hipEventDestroy(a);
            return -1;
        }
        P.pool[id].emplace_back(a, b);
    }
    const int idx = (int)P.used[id]++;
    (void)hipEventRecord(P.pool[id][idx].first, st);
    return idx;
}
void prof_stop(int id, int idx, hipStream_t st) {
    if (idx < 0) return;
    Profiler& P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    (void)hipEventRecord(P.pool[id][idx].second, st);
}
template <typename F>
hipError_t timed(int id, hipStream_t st, F&& launch, bool prof = true) {
    if (!prof) return launch();
    const int pi = prof_start(id, st);
    const hipError_t e = launch();
    prof_stop(id, pi, st);
    return e;
}

}  // namespace

// ----------------------------------------------------------------------------
// kernels local to this file
// ----------------------------------------------------------------------------
namespace kda {

int device_cu_count(int dev) {
    constexpr int MAXDEV = 64;
    static std::once_flag once[MAXDEV];
    static int cus[MAXDEV];
    if (dev < 0 || dev >= MAXDEV) return 0;
    std::call_once(once[dev], [dev] {
        int n = 0;
        cus[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) ? n : 0;
    });
    return cus[dev];
}

__global__ __launch_bounds__(256) void kda_state_copy_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                             size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src ? src[i] : 0.f;
}

hipError_t launch_state_copy(const float* src, float* dst, size_t n, hipStream_t st) {
    if (n == 0 || !dst) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(kda_state_copy_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st,
                       src, dst, n);
    return hipGetLastError();
}

// One workgroup per matrix: diagonal 16x16 inverses by substitution, then
// block substitution over 16-column tiles of b, fp32-accurate (split bf16) MFMA.
// The upper case solves the index-reversed (lower) system.
__global__ __launch_bounds__(256) void kda_solve_kernel(const float* __restrict__ M, const float* __restrict__ b,
                                                        float* __restrict__ y, int Cm, int N, int upper) {
    __shared__ float sl[C][C + 4];
    __shared__ float tii[NB][BS][BS + 4];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, g4 = l >> 4;
    const size_t mb = (size_t)blockIdx.x * Cm * Cm, bb = (size_t)blockIdx.x * Cm * N;
    const int nbk = (Cm + BS - 1) / BS;
    auto src = [&](int i) { return upper ? Cm - 1 - i : i; };
    for (int idx = tid; idx < C * C; idx += 256) {
        const int i = idx / C, j = idx - i * C;
        sl[i][j] = (i < Cm && j < i) ? M[mb + (size_t)src(i) * Cm + src(j)] : 0.f;
    }
    __syncthreads();
    diag_inverse<C + 4>(&sl[0][0], tii, nbk);
    __syncthreads();
    const int nct = (N + BS - 1) / BS;
    for (int ct = w; ct < nct; ct += 4) {
        const int col = ct * BS + r16;
        f32x4 X[NB];
        for (int i = 0; i < nbk; ++i) {
            f32x4 Y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = BS * i + 4 * g4 + e;
                Y[e] = (r < Cm && col < N) ? b[bb + (size_t)src(r) * N + col] : 0.f;
            }
            for (int j = 0; j < i; ++j) Y = mma4<3>(neg(frag4(&sl[0][0], C + 4, BS * i, BS * j)), acc2frag4(X[j]), Y);
            X[i] = mma4<3>(frag4(&tii[i][0][0], BS + 4, 0, 0), acc2frag4(Y), zero4());
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = BS * i + 4 * g4 + e;
                if (r < Cm && col < N) y[bb + (size_t)src(r) * N + col] = X[i][e];
            }
        }
    }
}

hipError_t launch_solve(const float* M, const float* b, float* y, int BH, int Cm, int N, int upper, hipStream_t st) {
    hipLaunchKernelGGL(kda_solve_kernel, dim3(BH), dim3(256), 0, st, M, b, y, Cm, N, upper);
    return hipGetLastError();
}

}  // namespace kda

// ----------------------------------------------------------------------------
// launch sequences
// ----------------------------------------------------------------------------
namespace {

bool valid_pass(int pass) { return pass == KDA_PASS_FWD || pass == KDA_PASS_BWD || pass == KDA_PASS_TRAIN; }

int check_workspace(const void* workspace, size_t ws_bytes, size_t need, const char* name = "workspace") {
    if (need == 0) return KDA_OK;
    if (!workspace || ws_bytes < need)
        return fail(KDA_E_WORKSPACE, "%s of %zu bytes given, %zu needed", name, workspace ? ws_bytes : 0, need);
    if (!aligned(workspace, 256)) return fail(KDA_E_INVALID, "%s is not 256-byte aligned", name);
    return KDA_OK;
}

// Prep: the forward's outputs (pass 0), the backward's (pass 1) or both (pass 2).
hipError_t launch_prep_pass(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
                            const Ws& ws, int T, int H, int D, int nchunks, int in_bf16, int g_kind,
                            hipStream_t st, bool prof = true, int dio = 0) {
    kda::PrepArgs pa = {};
    pa.dio = dio;
    pa.q = q; pa.k = k; pa.v = v; pa.g = g; pa.beta = beta;
    pa.W = region(ws, KDA_WS_W);
    pa.U = region(ws, KDA_WS_U);
    pa.KbT = region(ws, KDA_WS_KBT);
    pa.eG = fregion(ws, KDA_WS_EG);
    pa.Qp = region(ws, KDA_WS_QP);
    pa.Aqk = region(ws, KDA_WS_AQK);
    pa.WT = region(ws, KDA_WS_WT);
    pa.QpT = region(ws, KDA_WS_QPT);
    pa.Kb = region(ws, KDA_WS_KB);
    pa.AqkT = region(ws, KDA_WS_AQKT);
    pa.Akk = fregion(ws, KDA_WS_AKK);
    pa.Tii = fregion(ws, KDA_WS_TII);
    pa.T = T; pa.H = H; pa.nc = (T + kda::C - 1) / kda::C;
    const int id = pass == KDA_PASS_FWD ? PROF_PREP_FWD : pass == KDA_PASS_BWD ? PROF_PREP_BWD : PROF_PREP_TRAIN;
    return timed(id, st, [&] { return kda::launch_prep(pa, D, in_bf16, g_kind, nchunks, st); }, prof);
}

// The layer's gated RMSNorm fused into the forward's O store (kda_fwd_gated).
struct Epilogue {
    const void* z;
    int64_t ld_z;
    const float* w;
    float eps;
    void* y;
    int64_t ld_y;
};

// dio: the channels of a q, k, v, g (dout, dq, dk, dv, dg) row when narrower
// than D (0: D); dout_rec: the reverse carry's dout, D channels a row.
int fwd_launch(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
               const float* s0, void* o, float* s_final, int B, int T, int H, int D, int dtype, int g_dtype,
               const Ws& ws, hipStream_t st, bool prof, const Epilogue* epi, int dio = 0);
int bwd_launch(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
               const float* s0, const void* dout, const void* dout_rec, const float* ds_final, void* dq, void* dk,
               void* dv, void* dg, void* dbeta, float* ds0, int B, int T, int H, int D, int dtype, int g_dtype,
               const Ws& ws, hipStream_t st, int dio = 0);

// The padded head dimension's slots in the workspace's PAD and PADB regions,
// and the copies in and out of them.
struct PadIo {
    char *base, *base_b;
    PadLayout P;
    size_t ntok, nbh;
    int D, es;
    hipStream_t st;
    void* slot(int i) const { return (pad_backward_slot(i) ? base_b : base) + P.off[i]; }
    float* fslot(int i) const { return reinterpret_cast<float*>(slot(i)); }
    // the copies of one direction, gathered and issued as one launch: (B, T, H, D)
    // rows in / out (element size es) and (B, H, D, D) fp32 states in / out; a
    // null tensor adds nothing
    kda::ResizeJob jobs[kda::KDA_RESIZE_MAX_JOBS];
    int njobs = 0;
    void rows_in(const void* src, int i, int esz) { jobs[njobs++] = {src, slot(i), ntok, 1, D, 1, PAD_D, esz}; }
    void rows_out(int i, void* dst, int esz) { jobs[njobs++] = {slot(i), dst, ntok, 1, PAD_D, 1, D, esz}; }
    void state_in(const float* src, int i) {
        if (src) jobs[njobs++] = {src, slot(i), nbh, D, D, PAD_D, PAD_D, 4};
    }
    void state_out(int i, float* dst) {
        if (dst) jobs[njobs++] = {slot(i), dst, nbh, PAD_D, PAD_D, D, D, 4};
    }
    hipError_t issue() {
        const hipError_t e = kda::launch_resize_batch(jobs, njobs, st);
        njobs = 0;
        return e;
    }
};

PadIo pad_io(int pass, int B, int T, int H, int D, int dtype, const Ws& ws, hipStream_t st) {
    PadIo io;
    io.base = static_cast<char*>(ws.r[KDA_WS_PAD]);
    io.base_b = static_cast<char*>(ws.r[KDA_WS_PADB]);
    make_pad_layout(pass, B, T, H, dtype, io.P);
    io.ntok = (size_t)B * T * H;
    io.nbh = (size_t)B * H;
    io.D = D;
    io.es = (dtype == KDA_DTYPE_BF16) ? 2 : 4;
    io.st = st;
    return io;
}

int run_fwd_padded(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
                   const float* s0, void* o, float* s_final, int B, int T, int H, int D, int chunk, int dtype,
                   int g_dtype, const Ws& ws, hipStream_t st, bool prof) {
    PadIo io = pad_io(pass, B, T, H, D, dtype, ws, st);
    hipError_t e;
    io.state_in(s0, PS_S0);
    if ((e = io.issue()) != hipSuccess) return hip_fail(e, "kda_resize_batch_kernel (pad)");
    const int rc = fwd_launch(pass, q, k, v, g, beta, s0 ? io.fslot(PS_S0) : nullptr, io.slot(PS_O),
                              s_final ? io.fslot(PS_SF) : nullptr, B, T, H, PAD_D, dtype, g_dtype, ws, st, prof,
                              nullptr, D);
    if (rc != KDA_OK) return rc;
    io.rows_out(PS_O, o, io.es);
    io.state_out(PS_SF, s_final);
    if ((e = io.issue()) != hipSuccess) return hip_fail(e, "kda_resize_batch_kernel (crop)");
    return ok();
}

int run_bwd_padded(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
                   const float* s0, const void* dout, const float* ds_final, void* dq, void* dk, void* dv, void* dg,
                   void* dbeta, float* ds0, int B, int T, int H, int D, int dtype, int g_dtype, const Ws& ws,
                   hipStream_t st) {
    PadIo io = pad_io(pass, B, T, H, D, dtype, ws, st);
    hipError_t e;
    // the training backward finds the padded s0 where the training forward left
    // it (the pair's kept part is unmodified between the two calls, for the
    // same inputs)
    if (pass != KDA_PASS_TRAIN) io.state_in(s0, PS_S0);
    io.rows_in(dout, PS_DO, io.es);
    io.state_in(ds_final, PS_DSF);
    if ((e = io.issue()) != hipSuccess) return hip_fail(e, "kda_resize_batch_kernel (pad)");
    const int rc = bwd_launch(pass, q, k, v, g, beta, s0 ? io.fslot(PS_S0) : nullptr, dout, io.slot(PS_DO),
                              ds_final ? io.fslot(PS_DSF) : nullptr, dq, dk, dv, dg, dbeta,
                              ds0 ? io.fslot(PS_DS0) : nullptr, B, T, H, PAD_D, dtype, g_dtype, ws, st, D);
    if (rc != KDA_OK) return rc;
    io.state_out(PS_DS0, ds0);
    if ((e = io.issue()) != hipSuccess) return hip_fail(e, "kda_resize_batch_kernel (crop)");
    return ok();
}

// The forward's launch sequence (pass 0) or the training forward's (pass 2).
// prof = false: no launch timing, so the profiler's event pool never grows (for
// the entry point that must not allocate).
int run_fwd(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta, const float* s0,
            void* o, float* s_final, int B, int T, int H, int D, int chunk, int dtype, int g_dtype, void* workspace,
            size_t ws_bytes, void* stream, bool prof, const Epilogue* epi) {
    int rc = check_shape(B, T, H, D, chunk, dtype, g_dtype, pass == KDA_PASS_TRAIN);
    if (rc) return rc;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t nstate = (size_t)B * H * D * D;
    if ((rc = check_io(s0, "s0", KDA_DTYPE_F32, true)) || (rc = check_io(s_final, "s_final", KDA_DTYPE_F32, true)))
        return rc;
    if ((size_t)B * T * H == 0) {
        const hipError_t e = kda::launch_state_copy(s0, s_final, nstate, st);
        return e == hipSuccess ? ok() : hip_fail(e, "state copy");
    }
    if ((rc = check_io(q, "q", dtype, false)) || (rc = check_io(k, "k", dtype, false)) ||
        (rc = check_io(v, "v", dtype, false)) || (rc = check_io(g, "g", g_dtype, false)) ||
        (rc = check_io(o, "o", dtype, false)) || (rc = check_scalar(beta, "beta", dtype)))
        return rc;
    Layout L;
    make_layout(pass, B, T, H, D, dtype, L);
    // the training forward writes only the kept part of the pair's workspace
    if ((rc = check_workspace(workspace, ws_bytes, pass == KDA_PASS_TRAIN ? L.kept : L.total))) return rc;
    const Ws ws = resolve(L, workspace, nullptr);
    if (padded_head(D)) {
        if (epi) return fail(KDA_E_UNSUPPORTED, "D=%d has no fused epilogue", D);
        return run_fwd_padded(pass, q, k, v, g, beta, s0, o, s_final, B, T, H, D, chunk, dtype, g_dtype, ws, st,
                              prof);
    }
    return fwd_launch(pass, q, k, v, g, beta, s0, o, s_final, B, T, H, D, dtype, g_dtype, ws, st, prof, epi);
}

// The forward's launches on resolved workspace regions (shapes checked).
int fwd_launch(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
               const float* s0, void* o, float* s_final, int B, int T, int H, int D, int dtype, int g_dtype,
               const Ws& ws, hipStream_t st, bool prof, const Epilogue* epi, int dio) {
    const int nc = (T + kda::C - 1) / kda::C, BH = B * H;
    // g_dtype doubles as the launchers' g kind: 0 fp32, 1 bf16, 2 one fp32 decay per head
    const int in_bf16 = dtype == KDA_DTYPE_BF16, g_kind = g_dtype;
    hipError_t e =
        launch_prep_pass(pass, q, k, v, g, beta, ws, T, H, D, BH * nc, in_bf16, g_kind, st, prof, dio);
    if (e != hipSuccess) return hip_fail(e, "kda_prep_kernel");

    int nseg, seg_len;
    if (!epi && seg_forward(pass, B, T, H, D, dtype, &nseg, &seg_len)) {
        // bf16 D = 128, more than one segment: segment maps, start states, forward
        kda::SegArgs sa = {};
        sa.W = region(ws, KDA_WS_W);
        sa.U = region(ws, KDA_WS_U);
        sa.Qp = region(ws, KDA_WS_QP);
        sa.KbT = region(ws, KDA_WS_KBT);
        sa.Aqk = region(ws, KDA_WS_AQK);
        sa.eG = fregion(ws, KDA_WS_EG);
        sa.s0 = s0; sa.s_final = s_final; sa.o = o;
        if (pass == KDA_PASS_TRAIN) {
            // the training forward's own temporaries in the kept part
            if (!ws.segf) return fail(KDA_E_INVALID, "training forward over segments without its temporaries");
            sa.segX = reinterpret_cast<float*>(ws.segf);
            sa.segM = reinterpret_cast<uint16_t*>(ws.segf + ws.segf_per);
            sa.segS = reinterpret_cast<float*>(ws.segf + 2 * ws.segf_per);
        } else {
            sa.segX = fregion(ws, KDA_WS_SEGX);
            sa.segM = static_cast<uint16_t*>(region(ws, KDA_WS_SEGM));
            sa.segS = fregion(ws, KDA_WS_SEGS);
        }
        sa.T = T; sa.H = H; sa.nc = nc; sa.BH = BH; sa.nseg = nseg; sa.seg_len = seg_len;
        e = timed(PROF_SEG_MAP, st, [&] { return kda::launch_seg_map(sa, st); }, prof);
        if (e != hipSuccess) return hip_fail(e, "kda_segchain_kernel(map)");
        e = timed(PROF_SEG_SCAN, st, [&] { return kda::launch_seg_scan(sa, st); }, prof);
        if (e != hipSuccess) return hip_fail(e, "kda_segscan_kernel");
        e = timed(PROF_SEG_FWD, st, [&] { return kda::launch_seg_fwd(sa, st); }, prof);
        if (e != hipSuccess) return hip_fail(e, "kda_segchain_kernel(fwd)");
        return ok();
    }

    kda::RecurArgs ra = {};
    ra.W = region(ws, KDA_WS_W);
    ra.U = region(ws, KDA_WS_U);
    ra.Qp = region(ws, KDA_WS_QP);
    ra.KbT = region(ws, KDA_WS_KBT);
    ra.Kb = region(ws, KDA_WS_KB);
    ra.Aqk = region(ws, KDA_WS_AQK);
    ra.eG = fregion(ws, KDA_WS_EG);
    ra.s0 = s0; ra.s_final = s_final; ra.o = o;
    ra.T = T; ra.H = H; ra.nc = nc; ra.BH = BH;
    if (epi) {
        ra.z = epi->z; ra.ld_z = epi->ld_z; ra.nw = epi->w; ra.eps = epi->eps; ra.y = epi->y; ra.ld_y = epi->ld_y;
    }
    e = timed(PROF_RECUR_FWD, st, [&] { return kda::launch_recur(ra, D, in_bf16, 0, st); }, prof);
    if (e != hipSuccess) return hip_fail(e, "kda_recur_kernel");
    return ok();
}

// pass 1: prep from the inputs, then the backward; pass 2: the workspace holds
// the per-chunk factors kda_fwd_train wrote for the same inputs, so the prep is
// skipped.  Either way the chunk-boundary states are recomputed.
// scratch == nullptr: one workspace of the pass's whole layout; otherwise
// (pass 2 only) `workspace` holds the kept part and `scratch` the backward's.
int run_bwd(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta, const float* s0,
            const void* dout, const float* ds_final, void* dq, void* dk, void* dv, void* dg, void* dbeta, float* ds0,
            int B, int T, int H, int D, int chunk, int dtype, int g_dtype, const void* workspace, size_t ws_bytes,
            void* scratch, size_t scratch_bytes, bool split, void* stream) {
    int rc = check_shape(B, T, H, D, chunk, dtype, g_dtype, true);
    if (rc) return rc;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t nstate = (size_t)B * H * D * D;
    if ((rc = check_io(s0, "s0", KDA_DTYPE_F32, true)) || (rc = check_io(ds_final, "ds_final", KDA_DTYPE_F32, true)) ||
        (rc = check_io(ds0, "ds0", KDA_DTYPE_F32, true)))
        return rc;
    if ((size_t)B * T * H == 0) {
        const hipError_t e = kda::launch_state_copy(ds_final, ds0, nstate, st);
        return e == hipSuccess ? ok() : hip_fail(e, "state copy");
    }
    if ((rc = check_io(q, "q", dtype, false)) || (rc = check_io(k, "k", dtype, false)) ||
        (rc = check_io(v, "v", dtype, false)) || (rc = check_io(g, "g", g_dtype, false)) ||
        (rc = check_io(dout, "dout", dtype, false)) || (rc = check_io(dq, "dq", dtype, false)) ||
        (rc = check_io(dk, "dk", dtype, false)) || (rc = check_io(dv, "dv", dtype, false)) ||
        (rc = check_io(dg, "dg", g_dtype, false)) || (rc = check_scalar(beta, "beta", dtype)) ||
        (rc = check_scalar(dbeta, "dbeta", dtype)))
        return rc;
    Layout L;
    make_layout(pass, B, T, H, D, dtype, L);
    // the backward reads the kept part of a training workspace, never writes it
    void* kept = const_cast<void*>(workspace);
    Ws ws;
    if (split) {
        if ((rc = check_workspace(workspace, ws_bytes, L.kept)) ||
            (rc = check_workspace(scratch, scratch_bytes, L.total - L.kept, "scratch")))
            return rc;
        ws = resolve(L, kept, scratch);
    } else {
        if ((rc = check_workspace(workspace, ws_bytes, L.total))) return rc;
        ws = resolve(L, kept, static_cast<char*>(kept) + L.kept);
    }
    if (padded_head(D))
        return run_bwd_padded(pass, q, k, v, g, beta, s0, dout, ds_final, dq, dk, dv, dg, dbeta, ds0, B, T, H, D,
                              dtype, g_dtype, ws, st);
    return bwd_launch(pass, q, k, v, g, beta, s0, dout, dout, ds_final, dq, dk, dv, dg, dbeta, ds0, B, T, H, D,
                      dtype, g_dtype, ws, st);
}

// The backward's launches on resolved workspace regions (shapes checked).
int bwd_launch(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
               const float* s0, const void* dout, const void* dout_rec, const float* ds_final, void* dq, void* dk,
               void* dv, void* dg, void* dbeta, float* ds0, int B, int T, int H, int D, int dtype, int g_dtype,
               const Ws& ws, hipStream_t st, int dio) {
    const int nc = (T + kda::C - 1) / kda::C, BH = B * H;
    const int in_bf16 = dtype == KDA_DTYPE_BF16, g_kind = g_dtype;
    hipError_t e;
    if (pass == KDA_PASS_BWD) {
        e = launch_prep_pass(pass, q, k, v, g, beta, ws, T, H, D, BH * nc, in_bf16, g_kind, st, true, dio);
        if (e != hipSuccess) return hip_fail(e, "kda_prep_kernel");
    }
    void* W = region(ws, KDA_WS_W);
    void* U = region(ws, KDA_WS_U);
    void* KbT = region(ws, KDA_WS_KBT);
    float* eG = fregion(ws, KDA_WS_EG);
    void* hS = region(ws, KDA_WS_H);
    void* dhS = region(ws, KDA_WS_DH);
    void* Vp = region(ws, KDA_WS_VP);
    void* dVp = region(ws, KDA_WS_DVP);

    // chunk-boundary states, recomputed from the per-chunk factors: bf16 D = 128
    // over segments (maps, start states, the segments' chunk-start states),
    // otherwise one chain per (b, h)
    int nseg, seg_len;
    if (seg_states(pass, B, T, H, D, dtype, &nseg, &seg_len)) {
        kda::SegArgs sa = {};
        sa.W = W; sa.U = U; sa.KbT = KbT; sa.eG = eG; sa.s0 = s0; sa.h = hS; sa.Vp = Vp;
        sa.segX = fregion(ws, KDA_WS_SEGX);
        sa.segM = static_cast<uint16_t*>(region(ws, KDA_WS_SEGM));
        sa.segS = fregion(ws, KDA_WS_SEGS);
        sa.T = T; sa.H = H; sa.nc = nc; sa.BH = BH; sa.nseg = nseg; sa.seg_len = seg_len;
        sa.all_maps = 1;   // the reverse carry's scan below uses the last segment's map too
        e = timed(PROF_RECUR_H, st, [&] {
            hipError_t r = kda::launch_seg_map(sa, st);
            if (r == hipSuccess) r = kda::launch_seg_scan(sa, st);
            if (r == hipSuccess) r = kda::launch_seg_states(sa, st);
            return r;
        });
        if (e != hipSuccess) return hip_fail(e, "kda_segchain_kernel(states)");
    }
    // bf16 D = 128 without segments: the state recompute shares one launch with
    // the reverse carry below (kda_states_dh_kernel)
    const bool merged = nseg == 1 && in_bf16 && D == 128;
    kda::RecurArgs ra = {};
    if (nseg == 1) {
        ra.W = W; ra.U = U; ra.KbT = KbT; ra.eG = eG; ra.s0 = s0; ra.h = hS; ra.Vp = Vp;
        ra.Kb = region(ws, KDA_WS_KB);
        ra.T = T; ra.H = H; ra.nc = nc; ra.BH = BH;
        if (!merged) {
            e = timed(PROF_RECUR_H, st, [&] { return kda::launch_recur(ra, D, in_bf16, 1, st); });
            if (e != hipSuccess) return hip_fail(e, "kda_recur_kernel");
        }
    }

    kda::DhArgs da = {};
    da.AqkT = region(ws, KDA_WS_AQKT);
    da.Aqk = region(ws, KDA_WS_AQK);
    da.Qp = region(ws, KDA_WS_QP);
    da.W = W;
    da.Kb = region(ws, KDA_WS_KB);
    da.QpT = region(ws, KDA_WS_QPT);
    da.WT = region(ws, KDA_WS_WT);
    da.eG = eG; da.dout = dout_rec; da.dsf = ds_final; da.ds0 = ds0; da.dh = dhS; da.dVp = dVp;
    da.T = T; da.H = H; da.nc = nc; da.BH = BH;
    if (nseg > 1) {
        // the reverse carry over the recompute's segments: each segment's reverse
        // map (into segX, free after the recompute), the reverse scan from
        // ds_final through the forward maps' transposes (into segS), then every
        // segment's dh, dV' and dS0
        da.segX = fregion(ws, KDA_WS_SEGX);
        da.segS = fregion(ws, KDA_WS_SEGS);
        da.nseg = nseg;
        da.seg_len = seg_len;
        kda::SegArgs sr = {};
        sr.dsf = ds_final;
        sr.segX = da.segX;
        sr.segS = da.segS;
        sr.segM = static_cast<uint16_t*>(region(ws, KDA_WS_SEGM));
        sr.T = T; sr.H = H; sr.nc = nc; sr.BH = BH; sr.nseg = nseg; sr.seg_len = seg_len;
        e = timed(PROF_DH, st, [&] {
            hipError_t r = kda::launch_dh_seg_maps(da, st);
            if (r == hipSuccess) r = kda::launch_seg_rscan(sr, st);
            if (r == hipSuccess) r = kda::launch_dh_seg(da, st);
            return r;
        });
    } else if (merged) {
        e = timed(PROF_STATES_DH, st, [&] { return kda::launch_states_dh(ra, da, st); });
    } else {
        e = timed(PROF_DH, st, [&] { return kda::launch_dh(da, D, in_bf16, st); });
    }
    if (e != hipSuccess) return hip_fail(e, "kda_dh_kernel");

    kda::LocalArgs la = {};
    la.q = q; la.k = k; la.v = v; la.g = g; la.beta = beta; la.dout = dout;
    la.W = W; la.U = U; la.Akk = fregion(ws, KDA_WS_AKK); la.Tii = fregion(ws, KDA_WS_TII);
    la.h = hS; la.dh = dhS; la.Vp = Vp; la.dVp = dVp;
    la.dq = dq; la.dk = dk; la.dv = dv; la.dg = dg; la.dbeta = dbeta;
    la.T = T; la.H = H; la.nc = nc; la.dio = dio;
    e = timed(PROF_LOCAL, st, [&] { return kda::launch_local(la, D, in_bf16, g_kind, BH * nc, st); });
    if (e != hipSuccess) return hip_fail(e, "kda_bwd_local_kernel");
    return ok();
}

}  // namespace

// ----------------------------------------------------------------------------
// internal entry points for the other C-ABI translation units
// ----------------------------------------------------------------------------
namespace kda {

int api_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int api_hip_fail(hipError_t e, const char* where) { return hip_fail(e, where); }

size_t api_fwd_workspace_bytes(int B, int T, int H, int D, int chunk, int dtype, int g_dtype, int* rc) {
    *rc = check_shape(B, T, H, D, chunk, dtype, g_dtype, false);
    if (*rc != KDA_OK) return 0;
    Layout L;
    make_layout(KDA_PASS_FWD, B, T, H, D, dtype, L);
    return L.total;
}

int api_fwd_on_workspace(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const float* s0, void* o, float* s_final, int B, int T, int H, int D, int chunk, int dtype,
                         int g_dtype, void* workspace, size_t ws_bytes, void* stream) {
    return run_fwd(KDA_PASS_FWD, q, k, v, g, beta, s0, o, s_final, B, T, H, D, chunk, dtype, g_dtype, workspace,
                   ws_bytes, stream, /*prof=*/false, nullptr);
}

}  // namespace kda

// ----------------------------------------------------------------------------
// C ABI
// ----------------------------------------------------------------------------
extern "C" {

int kda_abi_version(void) { return 4; }

const char* kda_last_error(void) { return g_err.c_str(); }

size_t kda_workspace_size(int pass, int B, int T, int H, int D, int chunk, int dtype) {
    if (!valid_pass(pass)) {
        fail(KDA_E_INVALID, "pass=%d: expected 0 (fwd), 1 (bwd) or 2 (train)", pass);
        return 0;
    }
    if (check_shape(B, T, H, D, chunk, dtype, KDA_DTYPE_F32, pass != KDA_PASS_FWD) != KDA_OK) return 0;
    Layout L;
    make_layout(pass, B, T, H, D, dtype, L);
    ok();
    return L.total;
}

size_t kda_train_kept_size(int B, int T, int H, int D, int chunk, int dtype) {
    if (check_shape(B, T, H, D, chunk, dtype, KDA_DTYPE_F32, true) != KDA_OK) return 0;
    Layout L;
    make_layout(KDA_PASS_TRAIN, B, T, H, D, dtype, L);
    ok();
    return L.kept;
}

int kda_workspace_offsets(int pass, int B, int T, int H, int D, int chunk, int dtype, int64_t* offsets) {
    if (!offsets) return fail(KDA_E_INVALID, "offsets is NULL");
    if (!valid_pass(pass)) return fail(KDA_E_INVALID, "pass=%d", pass);
    const int rc = check_shape(B, T, H, D, chunk, dtype, KDA_DTYPE_F32, pass != KDA_PASS_FWD);
    if (rc) return rc;
    Layout L;
    make_layout(pass, B, T, H, D, dtype, L);
    for (int r = 0; r < KDA_WS_NREGIONS; ++r) offsets[r] = L.off[r];
    return ok();
}

int kda_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta, const float* s0, void* o,
            float* s_final, int B, int T, int H, int D, int chunk, int dtype, int g_dtype, void* workspace,
            size_t ws_bytes, void* stream) {
    return run_fwd(KDA_PASS_FWD, q, k, v, g, beta, s0, o, s_final, B, T, H, D, chunk, dtype, g_dtype, workspace,
                   ws_bytes, stream, true, nullptr);
}

int kda_fwd_train(const void* q, const void* k, const void* v, const void* g, const void* beta, const float* s0,
                  void* o, float* s_final, int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
                  void* workspace, size_t ws_bytes, void* stream) {
    return run_fwd(KDA_PASS_TRAIN, q, k, v, g, beta, s0, o, s_final, B, T, H, D, chunk, dtype, g_dtype, workspace,
                   ws_bytes, stream, true, nullptr);
}

int kda_fwd_gated(int pass, const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const float* s0, const void* z, int64_t ld_z, const float* norm_w, float eps, void* o, void* y,
                  int64_t ld_y, float* s_final, int B, int T, int H, int D, int chunk, int dtype, int g_dtype,
                  void* workspace, size_t ws_bytes, void* stream) {
    if (pass != KDA_PASS_FWD && pass != KDA_PASS_TRAIN)
        return fail(KDA_E_INVALID, "kda_fwd_gated: pass=%d, expected %d (forward) or %d (training)", pass,
                    KDA_PASS_FWD, KDA_PASS_TRAIN);
    int rc = check_shape(B, T, H, D, chunk, dtype, g_dtype, pass == KDA_PASS_TRAIN);
    if (rc) return rc;
    if (!kda::recur_epilogue_supported(D, dtype == KDA_DTYPE_BF16))
        return fail(KDA_E_UNSUPPORTED, "kda_fwd_gated: D=%d with dtype=%d has no fused epilogue (bf16: D=64; "
                    "fp32: D in {32, 64})", D, dtype);
    const int64_t epv = 16 / (dtype == KDA_DTYPE_BF16 ? 2 : 4);
    if ((size_t)B * T * H > 0) {
        if ((rc = check_io(z, "z", dtype, false)) || (rc = check_io(y, "y", dtype, false)) ||
            (rc = check_io(norm_w, "norm_w", KDA_DTYPE_F32, false)))
            return rc;
        if (ld_z < (int64_t)H * D || ld_z % epv || ld_y < (int64_t)H * D || ld_y % epv)
            return fail(KDA_E_INVALID, "kda_fwd_gated: ld_z=%lld and ld_y=%lld must be >= H*D=%d and multiples of %lld",
                        (long long)ld_z, (long long)ld_y, H * D, (long long)epv);
        if (!(eps >= 0.f)) return fail(KDA_E_INVALID, "kda_fwd_gated: eps=%g must be >= 0", (double)eps);
    }
    const Epilogue epi{z, ld_z, norm_w, eps, y, ld_y};
    return run_fwd(pass, q, k, v, g, beta, s0, o, s_final, B, T, H, D, chunk, dtype, g_dtype, workspace, ws_bytes,
                   stream, true, &epi);
}

int kda_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta, const float* s0,
            const void* dout, const float* ds_final, void* dq, void* dk, void* dv, void* dg, void* dbeta, float* ds0,
            int B, int T, int H, int D, int chunk, int dtype, int g_dtype, void* workspace, size_t ws_bytes,
            void* stream) {
    return run_bwd(KDA_PASS_BWD, q, k, v, g, beta, s0, dout, ds_final, dq, dk, dv, dg, dbeta, ds0, B, T, H, D, chunk,
                   dtype, g_dtype, workspace, ws_bytes, nullptr, 0, false, stream);
}

int kda_bwd_train(const void* q, const void* k, const void* v, const void* g, const void* beta, const float* s0,
                  const void* dout, const float* ds_final, void* dq, void* dk, void* dv, void* dg, void* dbeta,
                  float* ds0, int B, int T, int H, int D, int chunk, int dtype, int g_dtype, void* workspace,
                  size_t ws_bytes, void* stream) {
    return run_bwd(KDA_PASS_TRAIN, q, k, v, g, beta, s0, dout, ds_final, dq, dk, dv, dg, dbeta, ds0, B, T, H, D,
                   chunk, dtype, g_dtype, workspace, ws_bytes, nullptr, 0, false, stream);
}

int kda_bwd_train_split(const void* q, const void* k, const void* v, const void* g, const void* beta,
                        const float* s0, const void* dout, const float* ds_final, void* dq, void* dk, void* dv,
                        void* dg, void* dbeta, float* ds0, int B, int T, int H, int D, int chunk, int dtype,
                        int g_dtype, const void* kept, size_t kept_bytes, void* scratch, size_t scratch_bytes,
                        void* stream) {
    return run_bwd(KDA_PASS_TRAIN, q, k, v, g, beta, s0, dout, ds_final, dq, dk, dv, dg, dbeta, ds0, B, T, H, D,
                   chunk, dtype, g_dtype, kept, kept_bytes, scratch, scratch_bytes, true, stream);
}

int kda_solve_unit_triangular(const float* M, const float* b, float* y, int BH, int Cm, int N, int upper,
                              void* stream) {
    if (!M || !b || !y) return fail(KDA_E_INVALID, "M, b and y must be non-NULL");
    if (BH < 0 || N < 1 || Cm < 1) return fail(KDA_E_INVALID, "BH=%d Cm=%d N=%d", BH, Cm, N);
    if (Cm > kda::C) return fail(KDA_E_UNSUPPORTED, "Cm=%d exceeds 64", Cm);
    if (BH == 0) return ok();
    const hipError_t e = kda::launch_solve(M, b, y, BH, Cm, N, upper, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "kda_solve_kernel");
}

int kda_profile_enable(int on) {
    Profiler& P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    if (on)
        for (int i = 0; i < KDA_PROF_NKERNELS; ++i) P.used[i] = 0;
    P.on = on != 0;
    return ok();
}

const char* kda_profile_name(int id) {
    return (id >= 0 && id < KDA_PROF_NKERNELS) ? kProfNames[id] : "";
}

int kda_profile_read(int id, double* total_ms, int* launches) {
    if (id < 0 || id >= KDA_PROF_NKERNELS || !total_ms || !launches)
        return fail(KDA_E_INVALID, "kda_profile_read: bad arguments");
    Profiler& P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    double tot = 0.0;
    for (size_t i = 0; i < P.used[id]; ++i) {
        hipError_t e = hipEventSynchronize(P.pool[id][i].second);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, P.pool[id][i].first, P.pool[id][i].second);
        if (e != hipSuccess) return hip_fail(e, "kda_profile_read");
        tot += ms;
    }
    *total_ms = tot;
    *launches = (int)P.used[id];
    return ok();
}

}  // extern "C"

namespace {

// Activation rows are read and written four channels at a time.
int check_act(const void* p, const char* name, int dtype) {
    if (!p) return fail(KDA_E_INVALID, "%s is NULL", name);
    const size_t al = dtype == KDA_DTYPE_F32 ? 16 : 8;
    if (!aligned(p, al)) return fail(KDA_E_INVALID, "%s is not %zu-byte aligned", name, al);
    return KDA_OK;
}

int check_f32(const void* p, const char* name, size_t al, bool nullable) {
    if (!p) return nullable ? KDA_OK : fail(KDA_E_INVALID, "%s is NULL", name);
    if (!aligned(p, al)) return fail(KDA_E_INVALID, "%s is not %zu-byte aligned", name, al);
    return KDA_OK;
}

int check_ld(int64_t ld, int64_t min_ld, bool vec, const char* name) {
    if (ld < min_ld) return fail(KDA_E_INVALID, "%s=%lld is below the row width %lld", name, (long long)ld,
                                 (long long)min_ld);
    if (vec && ld % 4 != 0) return fail(KDA_E_INVALID, "%s=%lld is not a multiple of 4", name, (long long)ld);
    return KDA_OK;
}

int check_layer(int B, int T, int H, int D, int dtype, int g_dtype) {
    if (B < 0 || T < 0 || H < 1 || D < 1) return fail(KDA_E_INVALID, "B=%d T=%d H=%d D=%d", B, T, H, D);
    if (dtype != KDA_DTYPE_F32 && dtype != KDA_DTYPE_BF16)
        return fail(KDA_E_UNSUPPORTED, "dtype=%d: expected 0 (fp32) or 1 (bf16)", dtype);
    if (g_dtype != KDA_DTYPE_F32 && g_dtype != KDA_DTYPE_BF16)
        return fail(KDA_E_UNSUPPORTED, "g_dtype=%d: expected 0 (fp32) or 1 (bf16)", g_dtype);
    if (D % 4 != 0) return fail(KDA_E_UNSUPPORTED, "D=%d: must be a multiple of 4", D);
    if ((int64_t)H * D > 2048) return fail(KDA_E_UNSUPPORTED, "H*D=%d exceeds 2048", H * D);
    if ((int64_t)B * T > (int64_t)1 << 30) return fail(KDA_E_UNSUPPORTED, "B*T=%lld rows", (long long)B * T);
    return KDA_OK;
}

int check_norm(int rows, int H, int D, int dtype) {
    if (rows < 0 || H < 1 || D < 1) return fail(KDA_E_INVALID, "rows=%d H=%d D=%d", rows, H, D);
    if (dtype != KDA_DTYPE_F32 && dtype != KDA_DTYPE_BF16)
        return fail(KDA_E_UNSUPPORTED, "dtype=%d: expected 0 (fp32) or 1 (bf16)", dtype);
    if (D < 4 || D > 256 || D % 4 != 0)
        return fail(KDA_E_UNSUPPORTED, "D=%d: must be a multiple of 4 in [4, 256]", D);
    if ((int64_t)H * D > 2048) return fail(KDA_E_UNSUPPORTED, "H*D=%d exceeds 2048", H * D);
    if (kda::norm_waves(H, D) > 8)
        return fail(KDA_E_UNSUPPORTED, "H=%d heads of D=%d: more than 512 threads a row", H, D);
    return KDA_OK;
}

#define KDA_TRY(x) do { const int rc_ = (x); if (rc_ != KDA_OK) return rc_; } while (0)

int producer_common(const void* xq, const void* xk, const void* xv, const void* xf, const void* xb, int64_t ld_x,
                    int64_t ld_f, int64_t ld_b, const float* conv_w, const float* conv_b, const float* dt_bias,
                    const float* A_log, int B, int T, int H, int D, int dtype, int g_dtype) {
    KDA_TRY(check_layer(B, T, H, D, dtype, g_dtype));
    const int64_t HD = (int64_t)H * D;
    KDA_TRY(check_act(xq, "xq", dtype));
    KDA_TRY(check_act(xk, "xk", dtype));
    KDA_TRY(check_act(xv, "xv", dtype));
    KDA_TRY(check_scalar(xb, "xb", dtype));
    KDA_TRY(check_ld(ld_x, HD, true, "ld_x"));
    KDA_TRY(check_ld(ld_b, H, false, "ld_b"));
    KDA_TRY(check_f32(conv_w, "conv_w", 16, false));
    KDA_TRY(check_f32(conv_b, "conv_b", 16, true));
    // the decay gate (xf, dt_bias, A_log) is all present or all absent (scalar-alpha layer)
    if ((xf == nullptr) != (dt_bias == nullptr) || (xf == nullptr) != (A_log == nullptr))
        return fail(KDA_E_INVALID, "xf, dt_bias and A_log must be all NULL or all non-NULL");
    if (xf) {
        KDA_TRY(check_act(xf, "xf", dtype));
        KDA_TRY(check_ld(ld_f, HD, true, "ld_f"));
        KDA_TRY(check_f32(dt_bias, "dt_bias", 16, false));
        KDA_TRY(check_f32(A_log, "A_log", 4, false));
    }
    return KDA_OK;
}

}  // namespace

extern "C" {

int kda_layer_producer_fwd(const void* xq, const void* xk, const void* xv, const void* xf, const void* xb,
                           int64_t ld_x, int64_t ld_f, int64_t ld_b, const float* conv_w, const float* conv_b,
                           const float* dt_bias, const float* A_log, void* q, void* k, void* v, void* g, void* beta,
                           int B, int T, int H, int D, float scale, float beta_mult, int dtype, int g_dtype,
                           void* stream) {
    KDA_TRY(producer_common(xq, xk, xv, xf, xb, ld_x, ld_f, ld_b, conv_w, conv_b, dt_bias, A_log, B, T, H, D, dtype,
                            g_dtype));
    KDA_TRY(check_act(q, "q", dtype));
    KDA_TRY(check_act(k, "k", dtype));
    KDA_TRY(check_act(v, "v", dtype));
    if ((g == nullptr) != (xf == nullptr)) return fail(KDA_E_INVALID, "g must be NULL exactly when xf is NULL");
    if (g) KDA_TRY(check_act(g, "g", g_dtype));
    KDA_TRY(check_scalar(beta, "beta", dtype));
    if ((int64_t)B * T == 0) return ok();
    kda::ProdArgs a{};
    a.xq = xq; a.xk = xk; a.xv = xv; a.xf = xf; a.xb = xb;
    a.conv_w = conv_w; a.conv_b = conv_b; a.dt_bias = dt_bias; a.A_log = A_log;
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
    a.ld_x = ld_x; a.ld_f = ld_f; a.ld_b = ld_b;
    a.B = B; a.T = T; a.H = H; a.D = D; a.scale = scale; a.beta_mult = beta_mult;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = timed(PROF_PRODUCER_FWD, st, [&] {
        return kda::launch_producer_fwd(a, dtype == KDA_DTYPE_BF16, g_dtype == KDA_DTYPE_BF16, st);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "kda_layer_producer_fwd");
}

int kda_layer_producer_bwd(const void* xq, const void* xk, const void* xv, const void* xf, const void* xb,
                           int64_t ld_x, int64_t ld_f, int64_t ld_b, const float* conv_w, const float* conv_b,
                           const float* dt_bias, const float* A_log, const void* dq, const void* dk, const void* dv,
                           const void* dg, const void* dbeta, void* dxq, void* dxk, void* dxv, void* dxf, void* dxb,
                           int64_t ld_dx, int64_t ld_df, int64_t ld_db, float* dconv_w, float* dconv_b,
                           float* ddt_bias, float* dA_log, int B, int T, int H, int D, float scale, float beta_mult,
                           int dtype, int g_dtype, void* workspace, size_t ws_bytes, void* stream) {
    KDA_TRY(producer_common(xq, xk, xv, xf, xb, ld_x, ld_f, ld_b, conv_w, conv_b, dt_bias, A_log, B, T, H, D, dtype,
                            g_dtype));
    const int64_t HD = (int64_t)H * D;
    KDA_TRY(check_act(dq, "dq", dtype));
    KDA_TRY(check_act(dk, "dk", dtype));
    KDA_TRY(check_act(dv, "dv", dtype));
    if (xf) KDA_TRY(check_act(dg, "dg", g_dtype));
    KDA_TRY(check_scalar(dbeta, "dbeta", dtype));
    KDA_TRY(check_act(dxq, "dxq", dtype));
    KDA_TRY(check_act(dxk, "dxk", dtype));
    KDA_TRY(check_act(dxv, "dxv", dtype));
    if (xf) KDA_TRY(check_act(dxf, "dxf", dtype));
    KDA_TRY(check_scalar(dxb, "dxb", dtype));
    KDA_TRY(check_ld(ld_dx, HD, true, "ld_dx"));
    if (xf) KDA_TRY(check_ld(ld_df, HD, true, "ld_df"));
    KDA_TRY(check_ld(ld_db, H, false, "ld_db"));
    KDA_TRY(check_f32(dconv_w, "dconv_w", 4, false));
    if ((dg == nullptr) != (xf == nullptr) || (dxf == nullptr) != (xf == nullptr) ||
        (ddt_bias == nullptr) != (xf == nullptr) || (dA_log == nullptr) != (xf == nullptr))
        return fail(KDA_E_INVALID, "dg, dxf, ddt_bias and dA_log must be NULL exactly when xf is NULL");
    KDA_TRY(check_f32(ddt_bias, "ddt_bias", 4, true));
    KDA_TRY(check_f32(dA_log, "dA_log", 4, true));
    if ((conv_b == nullptr) != (dconv_b == nullptr))
        return fail(KDA_E_INVALID, "dconv_b must be NULL exactly when conv_b is NULL");
    KDA_TRY(check_f32(dconv_b, "dconv_b", 4, true));
    const size_t need = kda::producer_ws_floats(B, T, H, D) * sizeof(float);
    if (!workspace) return fail(KDA_E_INVALID, "workspace is NULL");
    if (!aligned(workspace, 16)) return fail(KDA_E_INVALID, "workspace is not 16-byte aligned");
    if (ws_bytes < need) return fail(KDA_E_WORKSPACE, "workspace has %zu bytes, needs %zu", ws_bytes, need);
    kda::ProdArgs a{};
    a.xq = xq; a.xk = xk; a.xv = xv; a.xf = xf; a.xb = xb;
    a.conv_w = conv_w; a.conv_b = conv_b; a.dt_bias = dt_bias; a.A_log = A_log;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.dbeta = dbeta;
    a.dxq = dxq; a.dxk = dxk; a.dxv = dxv; a.dxf = dxf; a.dxb = dxb;
    a.dconv_w = dconv_w; a.dconv_b = dconv_b; a.ddt_bias = ddt_bias; a.dA_log = dA_log;
    a.part = static_cast<float*>(workspace);
    a.colsum = a.part + (size_t)kda::producer_partials(B, T) * 17 * HD;
    a.ld_x = ld_x; a.ld_f = ld_f; a.ld_b = ld_b; a.ld_dx = ld_dx; a.ld_df = ld_df; a.ld_db = ld_db;
    a.B = B; a.T = T; a.H = H; a.D = D; a.scale = scale; a.beta_mult = beta_mult;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = timed(PROF_PRODUCER_BWD, st, [&] {
        return kda::launch_producer_bwd(a, dtype == KDA_DTYPE_BF16, g_dtype == KDA_DTYPE_BF16, st);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "kda_layer_producer_bwd");
}

int kda_layer_gated_rmsnorm_fwd(const void* o, const void* z, int64_t ld_z, const float* w, void* y, int64_t ld_y,
                                int rows, int H, int D, float eps, int dtype, void* stream) {
    KDA_TRY(check_norm(rows, H, D, dtype));
    const int64_t HD = (int64_t)H * D;
    KDA_TRY(check_act(o, "o", dtype));
    KDA_TRY(check_act(z, "z", dtype));
    KDA_TRY(check_act(y, "y", dtype));
    KDA_TRY(check_ld(ld_z, HD, true, "ld_z"));
    KDA_TRY(check_ld(ld_y, HD, true, "ld_y"));
    KDA_TRY(check_f32(w, "w", 16, false));
    if (rows == 0) return ok();
    kda::NormArgs a{};
    a.o = o; a.z = z; a.w = w; a.y = y; a.ld_z = ld_z; a.ld_y = ld_y;
    a.rows = rows; a.H = H; a.D = D; a.eps = eps;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = timed(PROF_RMSNORM_FWD, st, [&] { return kda::launch_rmsnorm_fwd(a, dtype == KDA_DTYPE_BF16, st); });
    return e == hipSuccess ? ok() : hip_fail(e, "kda_layer_gated_rmsnorm_fwd");
}

int kda_layer_gated_rmsnorm_bwd(const void* o, const void* z, int64_t ld_z, const float* w, const void* dy,
                                int64_t ld_dy, void* dout, void* dz, int64_t ld_dz, float* dw, int rows, int H, int D,
                                float eps, int dtype, void* workspace, size_t ws_bytes, void* stream) {
    KDA_TRY(check_norm(rows, H, D, dtype));
    const int64_t HD = (int64_t)H * D;
    KDA_TRY(check_act(o, "o", dtype));
    KDA_TRY(check_act(z, "z", dtype));
    KDA_TRY(check_act(dy, "dy", dtype));
    KDA_TRY(check_act(dout, "dout", dtype));
    KDA_TRY(check_act(dz, "dz", dtype));
    KDA_TRY(check_ld(ld_z, HD, true, "ld_z"));
    KDA_TRY(check_ld(ld_dy, HD, true, "ld_dy"));
    KDA_TRY(check_ld(ld_dz, HD, true, "ld_dz"));
    KDA_TRY(check_f32(w, "w", 16, false));
    KDA_TRY(check_f32(dw, "dw", 4, false));
    const size_t need = kda::rmsnorm_ws_floats(rows, H, D) * sizeof(float);
    if (!workspace) return fail(KDA_E_INVALID, "workspace is NULL");
    if (!aligned(workspace, 16)) return fail(KDA_E_INVALID, "workspace is not 16-byte aligned");
    if (ws_bytes < need) return fail(KDA_E_WORKSPACE, "workspace has %zu bytes, needs %zu", ws_bytes, need);
    kda::NormArgs a{};
    a.o = o; a.z = z; a.w = w; a.dy = dy; a.dout = dout; a.dz = dz; a.dw = dw;
    a.ld_z = ld_z; a.ld_dy = ld_dy; a.ld_dz = ld_dz;
    a.part = static_cast<float*>(workspace);
    a.colsum = a.part + (size_t)kda::rmsnorm_partials(rows) * HD;
    a.rows = rows; a.H = H; a.D = D; a.eps = eps;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = timed(PROF_RMSNORM_BWD, st, [&] { return kda::launch_rmsnorm_bwd(a, dtype == KDA_DTYPE_BF16, st); });
    return e == hipSuccess ? ok() : hip_fail(e, "kda_layer_gated_rmsnorm_bwd");
}

size_t kda_layer_workspace_size(int which, int B, int T, int H, int D) {
    if (B < 0 || T < 0 || H < 1 || D < 1) return 0;
    if (which == KDA_LAYER_PRODUCER) return kda::producer_ws_floats(B, T, H, D) * sizeof(float);
    if (which == KDA_LAYER_RMSNORM) return kda::rmsnorm_ws_floats(B * T, H, D) * sizeof(float);
    return 0;
}

}  // extern "C"
