// kda_internal.h -- kernel argument blocks and launcher declarations shared by
// the kernel translation units and the C-ABI layer.  Not installed.
//
// Workspace tensors, one slab per chunk (chunk id = (b*H + h)*nc + n).  Their
// element type ST is the input dtype (bf16 for bf16 inputs, fp32 for fp32
// inputs) except eG, Akk and Tii, which are always fp32:
//   W, U, Qp, Kb, Vp, dVp      [C][D]  row-major (token, channel)
//   WT, QpT, KbT               [D][C]  transposed copies for MFMA A operands
//                                      (bf16 D = 64: none of them; its kernels
//                                      read Kb, Qp, W, Aqk with transposing LDS
//                                      reads)
//   Aqk                        [C][C]  (token t, token s), zero above the diagonal
//   AqkT                       [C][C]  transpose of Aqk (not at bf16 D = 64)
//   Akk                        [C][C]  fp32, strictly lower, without the beta row scale
//   Tii                        [4][16][16] fp32 inverses of the diagonal blocks of I + L
//   eG                         [D]     fp32, e^{gamma of the chunk's last row}
//   h, dh                      [D][D]  state at chunk start / its adjoint at chunk end,
//                                      [dk][dv] orientation
#pragma once
#include <hip/hip_runtime.h>
#include <algorithm>
#include <type_traits>
#include "kda_chunk.h"

namespace kda {

struct PrepArgs {
    const void *q, *k, *v, *g, *beta;
    void *W, *U, *Qp, *QpT, *Kb, *KbT, *WT, *Aqk, *AqkT;
    float *Akk, *Tii, *eG;
    int T, H, nc;
    // channels of a q, k, v, g row when narrower than the kernel's D (D = 128
    // only, a multiple of 32; 0 = D): the missing channels are read as zero
    int dio;
};

struct RecurArgs {
    const void *W, *U, *Qp, *KbT, *Aqk;
    const void* Kb;   // bf16 D = 64 kernels read Kb (transposed in LDS) instead of Kb^T
    const float* eG;
    const float* s0;
    float* s_final;
    void* o;
    void *h, *Vp;
    int T, H, nc, BH;
    // h: mode 1 writes the chunk-start states there
    // Forward only: the layer's gated RMSNorm fused into the O store when y is
    // set, y = o rsqrt(mean_d o^2 + eps) nw sigmoid(z) per head; z and y are
    // [B, T, *] with row strides ld_z and ld_y (elements), head h at column h D.
    const void* z;
    const float* nw;
    void* y;
    int64_t ld_z, ld_y;
    float eps;
};

struct DhArgs {
    const void *AqkT, *Kb, *QpT, *WT;
    const void *Aqk, *Qp, *W;   // bf16 D = 64 reads these transposed instead of the T slabs
    const float* eG;
    const void* dout;
    const float* dsf;
    float* ds0;
    void *dh, *dVp;
    int T, H, nc, BH;
    // launch_dh_seg_maps / launch_dh_seg (bf16 D = 128): the segment plan, the
    // segments' reverse maps X_rev and incoming dSigma ([BH][nseg][D][D] fp32)
    float *segX, *segS;
    int nseg, seg_len;
};

struct LocalArgs {
    const void *q, *k, *v, *g, *beta, *dout;
    const void *W, *U, *h, *dh, *Vp, *dVp;
    const float *Akk, *Tii;
    void *dq, *dk, *dv, *dg, *dbeta;
    int T, H, nc;
    int pf_ahead;   // L2 prefetch distance in chunks (the device's CU count), 0 = none
    // channels of a q, k, v, g, dout, dq, dk, dv, dg row when narrower than the
    // kernel's D (the D = 128 kernel only, a multiple of 32; 0 = D): missing
    // channels are read as zero and not written
    int dio;
};

// The bf16 forward at D = 128 split over segments of the sequence (kda_seg.hip):
// pass A (launch_seg_map) writes each segment's map X, M; pass B
// (launch_seg_scan) the start state of segments 1 .. nseg - 1; pass C
// (launch_seg_fwd) O and the final state, or, for the backward's state
// recompute, (launch_seg_states) the chunk-start states h and V'.  segX, segS:
// [BH][nseg][D][D] fp32 in the reference orientation [dv][dk]; segM:
// [BH][nseg][2][D][D] bf16, M^T
// ([dk_in][dk_out]) split into hi and lo planes (the same bytes as fp32).
struct SegArgs {
    const void *W, *U, *Qp, *KbT, *Aqk;
    const float* eG;
    const float* s0;
    float* s_final;
    void* o;
    void *h, *Vp;   // launch_seg_states: chunk-start states [BH nc][D][D], V' [BH nc][C][D] (bf16)
    const float* dsf;   // launch_seg_rscan: ds_final (null: zero)
    int all_maps;       // launch_seg_map: the last segment's map too (the reverse scan's)
    float *segX, *segS;
    uint16_t* segM;
    int T, H, nc, BH, nseg, seg_len;
};
// segments for BH sequences of nc chunks: a function of the shape only
void seg_plan(int BH, int nc, int* nseg, int* seg_len);
hipError_t launch_seg_map(const SegArgs& a, hipStream_t st);
hipError_t launch_seg_scan(const SegArgs& a, hipStream_t st);
hipError_t launch_seg_fwd(const SegArgs& a, hipStream_t st);
hipError_t launch_seg_states(const SegArgs& a, hipStream_t st);
// The reverse scan of the backward's reverse carry over segments: from
// ds_final, dSigma entering segment s from its end, for s = nseg - 2 .. 0, as
// M_{s+1}^T dSigma_{s+1} + X_rev_{s+1} (segM from launch_seg_map with
// all_maps, segX the reverse maps), written to segS[s].
hipError_t launch_seg_rscan(const SegArgs& a, hipStream_t st);

// Compute-unit count of device `dev` (0 if it cannot be queried), looked up
// once per device under std::call_once, so concurrent callers are safe.
int device_cu_count(int dev);

// g_kind: 0 fp32 g [B, T, H, D], 1 bf16 g, 2 one fp32 decay per (b, t, h),
// g and dg [B, T, H] (GHead; bf16 inputs at D <= 64 only)
hipError_t launch_prep(const PrepArgs& a, int D, int in_bf16, int g_kind, int nchunks, hipStream_t st);
// mode 0: O and the final state (and y when a.y is set); 1: the chunk-start states h
hipError_t launch_recur(const RecurArgs& a, int D, int in_bf16, int mode, hipStream_t st);
// whether launch_recur can fuse the gated RMSNorm for this head size and dtype
bool recur_epilogue_supported(int D, int in_bf16);
hipError_t launch_dh(const DhArgs& a, int D, int in_bf16, hipStream_t st);
hipError_t launch_dh_seg_maps(const DhArgs& a, hipStream_t st);
// bf16 D = 128: the state recompute (MODE 1) and the reverse carry in one launch
hipError_t launch_states_dh(const RecurArgs& ra, const DhArgs& da, hipStream_t st);
hipError_t launch_dh_seg(const DhArgs& a, hipStream_t st);
hipError_t launch_local(const LocalArgs& a, int D, int in_bf16, int g_kind, int nchunks, hipStream_t st);
// the local adjoints at D = 128 (kda_bwdw.hip): reads A_kk, the diagonal-block
// inverses and V' from the workspace
hipError_t launch_local_wide(const LocalArgs& a, int D, int in_bf16, int g_bf16, int nchunks, hipStream_t st);
hipError_t launch_solve(const float* M, const float* b, float* y, int BH, int Cm, int N, int upper,
                        hipStream_t st);
hipError_t launch_state_copy(const float* src, float* dst, size_t n, hipStream_t st);
// Resize jobs (kda_pad.hip): n matrices of rs x cs elements (esize bytes each)
// into rd x cd, the common top-left block copied, the rest zero; up to
// KDA_RESIZE_MAX_JOBS of them in one launch (jobs with n = 0 skipped)
constexpr int KDA_RESIZE_MAX_JOBS = 8;
struct ResizeJob {
    const void* src;
    void* dst;
    size_t n;
    int rs, cs, rd, cd, esize;
};
hipError_t launch_resize_batch(const ResizeJob* jobs, int njobs, hipStream_t st);

// C-ABI helpers of kda_api.hip for the other C-ABI translation units (the
// allocation-free forward): the error setters behind kda_last_error(); the
// forward workspace size of a shape (0, with *rc the error code, for a shape
// the forward rejects); the forward's launch sequence on a given workspace,
// without launch timing.
int api_fail(int code, const char* fmt, ...);
int api_hip_fail(hipError_t e, const char* where);
size_t api_fwd_workspace_bytes(int B, int T, int H, int D, int chunk, int dtype, int g_dtype, int* rc);
int api_fwd_on_workspace(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const float* s0, void* o, float* s_final, int B, int T, int H, int D, int chunk, int dtype,
                         int g_dtype, void* workspace, size_t ws_bytes, void* stream);

// GatedDeltaLayer producer (projection outputs -> q, k, v, g, beta) and its
// adjoint.  Row strides are in elements; q, k, v, g, dq, dk, dv, dg are
// contiguous [B, T, H*D], beta and dbeta contiguous [B, T, H].
struct ProdArgs {
    const void *xq, *xk, *xv, *xf, *xb;
    const float *conv_w, *conv_b, *dt_bias, *A_log;   // [3][H*D][4], [3][H*D] or null, [H*D], [H]
    void *q, *k, *v, *g, *beta;
    const void *dq, *dk, *dv, *dg, *dbeta;
    void *dxq, *dxk, *dxv, *dxf, *dxb;
    float *dconv_w, *dconv_b, *ddt_bias, *dA_log;
    float *part, *colsum;                              // workspace
    int64_t ld_x, ld_f, ld_b, ld_dx, ld_df, ld_db;
    int B, T, H, D;
    float scale, beta_mult;
};

// Gated RMSNorm over heads of D channels; o and dout are contiguous [rows][H*D].
struct NormArgs {
    const void *o, *z, *dy;
    const float* w;
    void *y, *dout, *dz;
    float* dw;
    float *part, *colsum;                              // workspace
    int64_t ld_z, ld_y, ld_dy, ld_dz;
    int rows, H, D;
    float eps;
};

size_t producer_ws_floats(int B, int T, int H, int D);
size_t rmsnorm_ws_floats(int rows, int H, int D);
int producer_partials(int B, int T);
int rmsnorm_partials(int rows);
// waves of a norm workgroup: a head takes D / 4 lanes rounded up to a power of
// two (at most 8 waves: the kernels are bounded at 512 threads)
int norm_waves(int H, int D);
hipError_t launch_producer_fwd(const ProdArgs& a, int in_bf16, int g_bf16, hipStream_t st);
hipError_t launch_producer_bwd(const ProdArgs& a, int in_bf16, int g_bf16, hipStream_t st);
hipError_t launch_rmsnorm_fwd(const NormArgs& a, int in_bf16, hipStream_t st);
hipError_t launch_rmsnorm_bwd(const NormArgs& a, int in_bf16, hipStream_t st);

}  // namespace kda
