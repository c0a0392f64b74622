// kda_pad.hip -- head-dimension padding for D = 96.
//
// The chunk kernels tile the head dimension in 32- and 64-channel units, so a
// D = 96 call runs them at D = 128 with the channels 96..127 zero.  Zero
// channels change nothing in the first 96: a zero k (and q) channel keeps its
// state rows at zero and adds nothing to K K^T or Q K^T, a zero v channel
// keeps its state columns at zero, and g = 0 (no decay) there touches only
// those zero rows.  The outputs and gradients of the first 96 channels
// therefore equal the D = 96 recurrence's.  The prep and the local-adjoint
// kernel read and write 96-channel rows of q, k, v, g, dout and the gradients
// themselves; o, the reverse carry's dout and the states are padded or
// cropped here.
//
// kda_resize_batch_kernel: up to KDA_RESIZE_MAX_JOBS jobs in one launch; job j
// turns n matrices of rs x cs elements into rd x cd, element (r, c) of the
// output being the input's where r < rs and c < cs, else zero.  Padding
// (rd >= rs, cd >= cs) and cropping (rd <= rs, cd <= cs) are the same job.
// Rows move in 16-byte pieces (cs and cd are multiples of 16 bytes); the
// copies of one direction of a call (dout and the states in; o and the
// states out) go in one launch.
#include "kda_internal.h"

namespace kda {

namespace {

// Several resizes in one launch: job j owns workgroups [wg0[j], wg0[j + 1]),
// which stride over its n_pieces[j] destination pieces, so the job is uniform
// over a workgroup (its arguments stay scalar).
struct ResizeBatchArgs {
    const uint4* src[KDA_RESIZE_MAX_JOBS];
    uint4* dst[KDA_RESIZE_MAX_JOBS];
    size_t n_pieces[KDA_RESIZE_MAX_JOBS];
    int wg0[KDA_RESIZE_MAX_JOBS + 1];
    int rs[KDA_RESIZE_MAX_JOBS], cs[KDA_RESIZE_MAX_JOBS], rd[KDA_RESIZE_MAX_JOBS], cd[KDA_RESIZE_MAX_JOBS];
    int njobs;
};

__global__ __launch_bounds__(256) void kda_resize_batch_kernel(const ResizeBatchArgs a) {
    int j = 0;
    while (j + 1 < a.njobs && (int)blockIdx.x >= a.wg0[j + 1]) ++j;
    j = __builtin_amdgcn_readfirstlane(j);
    const uint4* __restrict__ src = a.src[j];
    uint4* __restrict__ dst = a.dst[j];
    const size_t total = a.n_pieces[j], per = (size_t)a.rd[j] * a.cd[j];
    const int rs = a.rs[j], cs = a.cs[j], cd = a.cd[j];
    const int nwg = a.wg0[j + 1] - a.wg0[j];
    for (size_t i = (size_t)(blockIdx.x - a.wg0[j]) * blockDim.x + threadIdx.x; i < total;
         i += (size_t)nwg * blockDim.x) {
        const size_t m = i / per;
        const int rem = (int)(i - m * per), r = rem / cd, c = rem - r * cd;
        uint4 x = make_uint4(0u, 0u, 0u, 0u);
        if (r < rs && c < cs) x = src[(m * rs + r) * cs + c];
        dst[i] = x;
    }
}

}  // namespace

hipError_t launch_resize_batch(const ResizeJob* jobs, int njobs, hipStream_t st) {
    if (njobs < 0 || njobs > KDA_RESIZE_MAX_JOBS) return hipErrorInvalidValue;
    ResizeBatchArgs a = {};
    int nj = 0, wg = 0;
    for (int j = 0; j < njobs; ++j) {
        const ResizeJob& b = jobs[j];
        if (b.n == 0) continue;
        if ((b.cs * b.esize) % 16 || (b.cd * b.esize) % 16) return hipErrorInvalidValue;
        a.src[nj] = static_cast<const uint4*>(b.src);
        a.dst[nj] = static_cast<uint4*>(b.dst);
        a.rs[nj] = b.rs;
        a.cs[nj] = b.cs * b.esize / 16;
        a.rd[nj] = b.rd;
        a.cd[nj] = b.cd * b.esize / 16;
        a.n_pieces[nj] = b.n * (size_t)a.rd[nj] * a.cd[nj];
        a.wg0[nj] = wg;
        // up to 2048 workgroups of 256 threads a job: each thread copies at
        // least one 16-byte piece, at most a few dozen
        wg += (int)std::min<size_t>((a.n_pieces[nj] + 255) / 256, 2048);
        ++nj;
    }
    a.wg0[nj] = wg;
    a.njobs = nj;
    if (wg == 0) return hipSuccess;
    hipLaunchKernelGGL(kda_resize_batch_kernel, dim3(wg), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace kda
