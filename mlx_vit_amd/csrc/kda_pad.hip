// kda_pad.hip -- head-dimension padding for D = 96.
//
// The chunk kernels tile the head dimension in 32- and 64-channel units, so a
// D = 96 call runs them at D = 128 on zero-padded copies.  Zero channels
// change nothing in the first 96: a zero k (and q) channel keeps its state
// rows at zero and adds nothing to K K^T or Q K^T, a zero v channel keeps its
// state columns at zero, and g = 0 (no decay) there touches only those zero
// rows.  The cropped outputs and gradients therefore equal the D = 96
// recurrence's.
//
// kda_resize_kernel: n matrices of rs x cs elements into rd x cd; element
// (r, c) of the output is the input's where r < rs and c < cs, else zero.
// Padding (rd >= rs, cd >= cs) and cropping (rd <= rs, cd <= cs) are the same
// kernel.  Rows move in 16-byte pieces (cs and cd are multiples of 16 bytes).
#include "kda_internal.h"

namespace kda {

namespace {

__global__ __launch_bounds__(256) void kda_resize_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         size_t n, int rs, int cs, int rd, int cd) {
    // cs, cd: row lengths in 16-byte pieces
    const size_t per = (size_t)rd * cd, total = n * per;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t m = i / per;
        const int rem = (int)(i - m * per), r = rem / cd, c = rem - r * cd;
        uint4 x = make_uint4(0u, 0u, 0u, 0u);
        if (r < rs && c < cs) x = src[(m * rs + r) * cs + c];
        dst[i] = x;
    }
}

}  // namespace

hipError_t launch_resize(const void* src, void* dst, size_t n, int rs, int cs, int rd, int cd, int esize,
                         hipStream_t st) {
    if (n == 0) return hipSuccess;
    if ((cs * esize) % 16 || (cd * esize) % 16) return hipErrorInvalidValue;
    const int cs16 = cs * esize / 16, cd16 = cd * esize / 16;
    const size_t total = n * (size_t)rd * cd16;
    const unsigned grid = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(kda_resize_kernel, dim3(grid), dim3(256), 0, st, static_cast<const uint4*>(src),
                       static_cast<uint4*>(dst), n, rs, cs16, rd, cd16);
    return hipGetLastError();
}

}  // namespace kda
