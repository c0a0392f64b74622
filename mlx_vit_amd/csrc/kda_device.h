// kda_device.h -- device-side building blocks shared by the gfx950 KDA kernels.
//
// Wave64 MFMA conventions (gfx950, verified on hardware):
//   v_mfma_f32_16x16x32_bf16   A: lane l holds row (l % 16), k-slots 8*(l/16)+e, e = 0..7
//                              B: lane l holds col (l % 16), same k-slots
//                              D: lane l holds col (l % 16), rows 4*(l/16)+i, i = 0..3
//   v_mfma_f32_16x16x16_bf16   as above with k-slots 4*(l/16)+e, e = 0..3
//
// K permutation.  A contraction does not care which physical k a slot holds as
// long as A and B agree.  Every 32-wide k-step here maps slot (g = l/16, e) to
//     k = (e < 4) ? 4g + e : 16 + 4g + (e - 4)
// which is exactly how two stacked 16-row accumulator tiles are spread over the
// lanes.  So any accumulator pair (rows k0..k0+31 of a product) can be fed back
// as the B operand of the next MFMA with no data movement, and every operand
// read from memory is a pair of 4-element vectors at k0+4g and k0+16+4g.
//
// Precision.  PREC == 1 rounds both operands to bf16 (one MFMA).  PREC == 3
// splits each fp32 operand into hi + lo bf16 parts and issues hi*hi + hi*lo +
// lo*hi, which carries ~16 mantissa bits (relative error ~1e-5); it is used for
// fp32 inputs and for the small triangular-solve products.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int C = 64;       // chunk length (tokens)
constexpr int BS = 16;      // sub-block edge = MFMA tile edge
constexpr int NB = C / BS;  // sub-blocks per chunk
constexpr float SPAN_MAX = 60.0f;  // largest in-block decay span the anchored MFMA path accepts

// ----------------------------------------------------------------------------
// scalar conversions (bf16 is carried as raw uint16_t bits)
// ----------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);                                           // round to nearest even
    return (uint16_t)(u >> 16);
}

template <typename T> __device__ __forceinline__ float ld1(const T* p);
template <> __device__ __forceinline__ float ld1<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld1<uint16_t>(const uint16_t* p) { return bf2f(*p); }

template <typename T> __device__ __forceinline__ void st1(T* p, float v);
template <> __device__ __forceinline__ void st1<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void st1<uint16_t>(uint16_t* p, float v) { *p = f2bf(v); }

// four consecutive elements -> float4
template <typename T> __device__ __forceinline__ float4 ld4(const T* p);
template <> __device__ __forceinline__ float4 ld4<float>(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}
template <> __device__ __forceinline__ float4 ld4<uint16_t>(const uint16_t* p) {
    uint2 r = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                       __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ----------------------------------------------------------------------------
// fragments: 8 (or 4) fp32 k-slot values per lane, converted at MFMA time
// ----------------------------------------------------------------------------
struct Fr8 { float v[8]; };
struct Fr4 { float v[4]; };

__device__ __forceinline__ void split_bf16(float x, __bf16& hi, __bf16& lo) {
    hi = (__bf16)x;
    lo = (__bf16)(x - (float)hi);
}

template <int PREC>
__device__ __forceinline__ f32x4 mma8(const Fr8& a, const Fr8& b, f32x4 c) {
    if constexpr (PREC == 1) {
        bf16x8 A, B;
#pragma unroll
        for (int e = 0; e < 8; ++e) { A[e] = (__bf16)a.v[e]; B[e] = (__bf16)b.v[e]; }
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, c, 0, 0, 0);
    } else {
        bf16x8 Ah, Al, Bh, Bl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            __bf16 h, l;
            split_bf16(a.v[e], h, l); Ah[e] = h; Al[e] = l;
            split_bf16(b.v[e], h, l); Bh[e] = h; Bl[e] = l;
        }
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bh, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bl, c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bh, c, 0, 0, 0);
    }
}

__device__ __forceinline__ short4v pack4(const float* v) {
    short4v r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (short)f2bf(v[e]);
    return r;
}

template <int PREC>
__device__ __forceinline__ f32x4 mma4(const Fr4& a, const Fr4& b, f32x4 c) {
    if constexpr (PREC == 1) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(a.v), pack4(b.v), c, 0, 0, 0);
    } else {
        float ah[4], al[4], bh[4], bl[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ah[e] = bf2f(f2bf(a.v[e])); al[e] = a.v[e] - ah[e];
            bh[e] = bf2f(f2bf(b.v[e])); bl[e] = b.v[e] - bh[e];
        }
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(al), pack4(bh), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(ah), pack4(bl), c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(ah), pack4(bh), c, 0, 0, 0);
    }
}

// k index of slot e for lane group g (32-wide k-step)
__device__ __forceinline__ int kslot(int g, int e) { return (e < 4) ? (4 * g + e) : (16 + 4 * g + e - 4); }

// Row-major operand, k contiguous: lane reads row (row0 + l%16), k-slots of the
// 32-wide step starting at k0.  Works for fp32 or bf16 storage, LDS or global.
template <typename T>
__device__ __forceinline__ Fr8 frag8(const T* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    const T* p = M + (size_t)(row0 + r) * ld + k0 + 4 * g;
    float4 x = ld4<T>(p), y = ld4<T>(p + 16);
    Fr8 f;
    f.v[0] = x.x; f.v[1] = x.y; f.v[2] = x.z; f.v[3] = x.w;
    f.v[4] = y.x; f.v[5] = y.y; f.v[6] = y.z; f.v[7] = y.w;
    return f;
}

// 16-wide k-step: lane reads row (row0 + l%16), k = k0 + 4g + 0..3
template <typename T>
__device__ __forceinline__ Fr4 frag4(const T* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    float4 x = ld4<T>(M + (size_t)(row0 + r) * ld + k0 + 4 * g);
    Fr4 f;
    f.v[0] = x.x; f.v[1] = x.y; f.v[2] = x.z; f.v[3] = x.w;
    return f;
}

// 16-wide k-step of the TRANSPOSE of a row-major matrix: A[row][k] = M[k][row]
__device__ __forceinline__ Fr4 frag4T(const float* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    Fr4 f;
#pragma unroll
    for (int e = 0; e < 4; ++e) f.v[e] = M[(size_t)(k0 + 4 * g + e) * ld + row0 + r];
    return f;
}

// accumulator pair (rows k0..k0+15, k0+16..k0+31 of some product) as a B operand
__device__ __forceinline__ Fr8 acc2frag(const f32x4& lo, const f32x4& hi) {
    Fr8 f;
#pragma unroll
    for (int e = 0; e < 4; ++e) { f.v[e] = lo[e]; f.v[4 + e] = hi[e]; }
    return f;
}
__device__ __forceinline__ Fr4 acc2frag4(const f32x4& a) {
    Fr4 f;
#pragma unroll
    for (int e = 0; e < 4; ++e) f.v[e] = a[e];
    return f;
}

__device__ __forceinline__ Fr8 neg(Fr8 f) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f.v[e] = -f.v[e];
    return f;
}
__device__ __forceinline__ Fr4 neg(Fr4 f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f.v[e] = -f.v[e];
    return f;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// ----------------------------------------------------------------------------
// XCD-aware block remap: blocks with equal blockIdx % 8 run on one XCD (one
// L2).  Renumber so that a run of `group` consecutive logical blocks (the dv
// tiles of one (batch, head)) shares an XCD.  Identity when the grid does not
// split evenly.
// ----------------------------------------------------------------------------
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int NXCD = 8;
    if (nblocks % NXCD != 0) return bid;
    return (bid % NXCD) * (nblocks / NXCD) + bid / NXCD;
}

}  // namespace kda
