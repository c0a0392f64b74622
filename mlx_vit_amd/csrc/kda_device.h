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
// fp32 inputs and for the small triangular-solve products.  PREC == 2 splits
// only A (hi*hi + lo*hi), for products whose B operand is exact in bf16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

namespace kda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int C = 64;       // chunk length (tokens)
constexpr int BS = 16;      // sub-block edge = MFMA tile edge
constexpr int NB = C / BS;  // sub-blocks per chunk
constexpr float SPAN_MAX = 60.0f;  // largest in-block decay span the anchored MFMA path accepts
// largest 4-row decay span the sub-anchored diagonal tiles accept: their
// operands reach e^{span} |k|, e^80 |k| staying far inside the fp32 / bf16 range
constexpr float SUB_SPAN_MAX = 80.0f;

// ----------------------------------------------------------------------------
// scalar conversions (bf16 is carried as raw uint16_t bits)
// ----------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// round to nearest even (v_cvt_pk_bf16_f32; NaN stays NaN)
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two floats to a packed bf16 pair, a in the low half: one v_cvt_pk_bf16_f32
// with both sources (converting each alone and merging the halves costs four
// VALU operations).  Same rounding as f2bf.
__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
// the two halves of a packed pair back as floats
__device__ __forceinline__ float bf_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
// packed pair of (v - the value of v's bf16 pair): the lo parts of a bf16 hi + lo split
__device__ __forceinline__ uint32_t pack2bf_rest(float a, float b, uint32_t h) {
    return pack2bf(a - bf_lo(h), b - bf_hi(h));
}

// Element-type tag of a decay given once per (batch, token, head): fp32
// [B, T, H], shared by the head's D channels (the scalar-alpha GDN, g = log
// alpha).  Its gradient is the sum over the channels, fp32 [B, T, H] too.
struct GHead {};

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
        const uint4 A = make_uint4(pack2bf(a.v[0], a.v[1]), pack2bf(a.v[2], a.v[3]), pack2bf(a.v[4], a.v[5]),
                                   pack2bf(a.v[6], a.v[7]));
        const uint4 B = make_uint4(pack2bf(b.v[0], b.v[1]), pack2bf(b.v[2], b.v[3]), pack2bf(b.v[4], b.v[5]),
                                   pack2bf(b.v[6], b.v[7]));
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A), __builtin_bit_cast(bf16x8, B), c,
                                                       0, 0, 0);
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
    return __builtin_bit_cast(short4v, make_uint2(pack2bf(v[0], v[1]), pack2bf(v[2], v[3])));
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
        // PREC 4 also adds lo * lo: the product of the split operands is then
        // exact, so two MFMAs that share a split operand agree to fp32
        if constexpr (PREC >= 4) c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(al), pack4(bl), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(al), pack4(bh), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(ah), pack4(bl), c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack4(ah), pack4(bh), c, 0, 0, 0);
    }
}

// The value an MFMA of precision PREC effectively multiplies for the fp32
// operand v: bf16(v) at PREC 1, bf16(v) + bf16(v - bf16(v)) with the split.
template <int PREC>
__device__ __forceinline__ float mfma_operand(float v) {
    const float hi = bf2f(f2bf(v));
    if constexpr (PREC == 1) return hi;
    else return hi + bf2f(f2bf(v - hi));
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
// bf16-native operands: raw bf16 bits in memory go straight into the MFMA
// (no fp32 round trip).  Frag8 carries a hi part and, for PREC >= 2, a lo part.
// ----------------------------------------------------------------------------
struct Frag8 { bf16x8 h, l; };
struct Frag4 { short4v h, l; };

// hi = bf16(v), lo = bf16(v - hi) (PREC >= 2), converted a pair at a time
template <int PREC>
__device__ __forceinline__ Frag8 frag_from_f32(const float* v) {
    Frag8 f;
    uint32_t h[4], lo[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        h[p] = pack2bf(v[2 * p], v[2 * p + 1]);
        if constexpr (PREC >= 2) lo[p] = pack2bf_rest(v[2 * p], v[2 * p + 1], h[p]);
    }
    f.h = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
    f.l = __builtin_bit_cast(bf16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
    return f;
}

template <int PREC>
__device__ __forceinline__ Frag4 frag4_from_f32(const float* v) {
    Frag4 f;
    const uint32_t h0 = pack2bf(v[0], v[1]), h1 = pack2bf(v[2], v[3]);
    f.h = __builtin_bit_cast(short4v, make_uint2(h0, h1));
    if constexpr (PREC >= 2)
        f.l = __builtin_bit_cast(short4v, make_uint2(pack2bf_rest(v[0], v[1], h0), pack2bf_rest(v[2], v[3], h1)));
    else
        f.l = short4v{0, 0, 0, 0};
    return f;
}

// A operand (row-major, k contiguous) or B operand stored n-major, k contiguous.
template <int PREC, typename ST>
__device__ __forceinline__ Frag8 ldfrag(const ST* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    const ST* p = M + (size_t)(row0 + r) * ld + k0 + 4 * g;
    if constexpr (std::is_same<ST, uint16_t>::value) {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        const uint2 y = *reinterpret_cast<const uint2*>(p + 16);
        Frag8 f;
        f.h = __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
        if constexpr (PREC >= 2) f.l = __builtin_bit_cast(bf16x8, make_uint4(0u, 0u, 0u, 0u));
        return f;
    } else {
        const float4 x = *reinterpret_cast<const float4*>(p);
        const float4 y = *reinterpret_cast<const float4*>(p + 16);
        const float v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
        return frag_from_f32<PREC>(v);
    }
}

// ldfrag with the hardware's own k-slot order instead of the K permutation:
// slot (g, e) holds k = k0 + 8 g + e, so a lane's eight elements are one
// contiguous 16-byte piece (bf16; two for fp32).  Only for products whose A
// and B operands both come from memory rows this way -- never with an
// accumulator fed back as B, which carries the K permutation.  With rows
// 16 bytes mod 128 apart (a 16-byte row pad), the eight lanes of a 16-byte
// LDS read hit eight distinct bank groups.
template <int PREC, typename ST>
__device__ __forceinline__ Frag8 ldfrag_c(const ST* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    const ST* p = M + (size_t)(row0 + r) * ld + k0 + 8 * g;
    if constexpr (std::is_same<ST, uint16_t>::value) {
        Frag8 f;
        f.h = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
        if constexpr (PREC >= 2) f.l = __builtin_bit_cast(bf16x8, make_uint4(0u, 0u, 0u, 0u));
        return f;
    } else {
        const float4 x = *reinterpret_cast<const float4*>(p);
        const float4 y = *reinterpret_cast<const float4*>(p + 4);
        const float v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
        return frag_from_f32<PREC>(v);
    }
}
// ldfrag_c with every k-slot multiplied by scale[k - k0]
template <int PREC, typename ST>
__device__ __forceinline__ Frag8 ldfrag_c_scaled(const ST* M, int ld, int row0, int k0, const float* scale) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    const ST* p = M + (size_t)(row0 + r) * ld + k0 + 8 * g;
    const float4 x = ld4<ST>(p), y = ld4<ST>(p + 4);
    const float4 sx = *reinterpret_cast<const float4*>(scale + 8 * g);
    const float4 sy = *reinterpret_cast<const float4*>(scale + 8 * g + 4);
    const float v[8] = {x.x * sx.x, x.y * sx.y, x.z * sx.z, x.w * sx.w, y.x * sy.x, y.y * sy.y, y.z * sy.z, y.w * sy.w};
    return frag_from_f32<PREC>(v);
}

// 16-wide k-step, row-major k contiguous
template <int PREC, typename ST>
__device__ __forceinline__ Frag4 ldfrag4(const ST* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    const ST* p = M + (size_t)(row0 + r) * ld + k0 + 4 * g;
    if constexpr (std::is_same<ST, uint16_t>::value) {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        Frag4 f;
        f.h = __builtin_bit_cast(short4v, x);
        if constexpr (PREC >= 2) f.l = short4v{0, 0, 0, 0};
        return f;
    } else {
        const float4 x = *reinterpret_cast<const float4*>(p);
        const float v[4] = {x.x, x.y, x.z, x.w};
        return frag4_from_f32<PREC>(v);
    }
}

// 16-wide k-step of the transpose: A[row][k] = M[k][row]
template <int PREC, typename ST>
__device__ __forceinline__ Frag4 ldfrag4T(const ST* M, int ld, int row0, int k0) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = ld1<ST>(M + (size_t)(k0 + 4 * g + e) * ld + row0 + r);
    return frag4_from_f32<PREC>(v);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  In each group of 16
// lanes the sixteen 8-byte pieces the lanes address are 64 16-bit elements in
// lane order (the piece of lane j holds positions 4 j .. 4 j + 3), and lane i
// of the group receives positions i, 16 + i, 32 + i, 48 + i.  So when lane j of
// group g addresses row k0 + 4 g + j / 4, columns n0 + 4 (j % 4) .. + 3 of a
// row-major bf16 tile M[k][n], lane (n = i, g) receives M[k0 + 4 g + e][n0 + i],
// e = 0..3: the k-slots 4 g .. 4 g + 3 of an MFMA operand that is stored with k
// along the rows (the lane layout was checked on the device with in-bounds
// addresses).  Each address must be 8-byte aligned.
typedef __attribute__((address_space(3))) short4v lds_short4v;
__device__ __forceinline__ short4v ld_tr4(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(const_cast<uint16_t*>(p)));
}
// B fragment (16x16x32, ldfrag's k-slot order) B[k][n] = M[k0 + k][n0 + n] of a
// row-major bf16 tile whose rows are k (row stride ld elements)
__device__ __forceinline__ Frag8 ldfragT(const uint16_t* M, int ld, int n0, int k0) {
    const int l = lane_id(), j = l & 15, g = l >> 4;
    const uint16_t* p = M + (size_t)(k0 + 4 * g + (j >> 2)) * ld + n0 + 4 * (j & 3);
    const short4v x = ld_tr4(p), y = ld_tr4(p + (size_t)16 * ld);
    Frag8 f;
    f.h = __builtin_bit_cast(bf16x8, short8v{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]});
    return f;
}
// Eight consecutive rows of one column of an [n][ld] bf16 LDS tile X, for
// writing its transpose as 16-byte row pieces: lane i of each 16-lane group
// receives X[n0 + 8 (i / 4) + c][k0 + i % 4], c = 0..7, with two transposing
// reads (the group covers columns k0..k0+3 of rows n0..n0+31).  Rows of X
// must be 8-byte aligned at column k0.
__device__ __forceinline__ short8v ld_tr_rows8(const uint16_t* X, int ld, int n0, int k0) {
    const int j = lane_id() & 15;
    const uint16_t* p = X + (size_t)(n0 + 8 * (j & 3) + (j >> 2)) * ld + k0;
    const short4v x = ld_tr4(p), y = ld_tr4(p + (size_t)4 * ld);
    return short8v{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

// the same for a 16x16x16 operand (k-slots 4 g .. 4 g + 3)
__device__ __forceinline__ Frag4 ldfrag4T_tr(const uint16_t* M, int ld, int n0, int k0) {
    const int l = lane_id(), j = l & 15, g = l >> 4;
    Frag4 f;
    f.h = ld_tr4(M + (size_t)(k0 + 4 * g + (j >> 2)) * ld + n0 + 4 * (j & 3));
    return f;
}
// four rows k0 + 4 g + e, e = 0..3, of column n0 + (l % 16) as floats
__device__ __forceinline__ void ld_col4(const uint16_t* M, int ld, int n0, int k0, float* v) {
    const int l = lane_id(), j = l & 15, g = l >> 4;
    const short4v x = ld_tr4(M + (size_t)(k0 + 4 * g + (j >> 2)) * ld + n0 + 4 * (j & 3));
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = bf2f((uint16_t)x[e]);
}

// ldfrag with every k-slot multiplied by scale[k - k0]
template <int PREC, typename ST>
__device__ __forceinline__ Frag8 ldfrag_scaled(const ST* M, int ld, int row0, int k0, const float* scale) {
    const int l = lane_id(), r = l & 15, g = l >> 4;
    const ST* p = M + (size_t)(row0 + r) * ld + k0 + 4 * g;
    const float4 x = ld4<ST>(p), y = ld4<ST>(p + 16);
    const float4 sx = *reinterpret_cast<const float4*>(scale + 4 * g);
    const float4 sy = *reinterpret_cast<const float4*>(scale + 16 + 4 * g);
    const float v[8] = {x.x * sx.x, x.y * sx.y, x.z * sx.z, x.w * sx.w, y.x * sy.x, y.y * sy.y, y.z * sy.z, y.w * sy.w};
    return frag_from_f32<PREC>(v);
}

template <int PREC>
__device__ __forceinline__ Frag8 accfrag(const f32x4& lo, const f32x4& hi) {
    const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return frag_from_f32<PREC>(v);
}
template <int PREC>
__device__ __forceinline__ Frag4 accfrag4(const f32x4& a) {
    const float v[4] = {a[0], a[1], a[2], a[3]};
    return frag4_from_f32<PREC>(v);
}

template <int PREC>
__device__ __forceinline__ f32x4 mma(const Frag8& a, const Frag8& b, f32x4 c) {
    // PREC 3: both operands split into bf16 hi + lo; PREC 2: only A split (B is
    // exact in bf16, its lo part is zero); PREC 1: bf16 operands
    if constexpr (PREC >= 2) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.l, b.h, c, 0, 0, 0);
    if constexpr (PREC == 3) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.l, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.h, c, 0, 0, 0);
}
// [x | y]: two 4-element fragments as the two k-halves of one 8-element fragment
__device__ __forceinline__ bf16x8 cat4(short4v x, short4v y) {
    const uint2 u = __builtin_bit_cast(uint2, x), v = __builtin_bit_cast(uint2, y);
    return __builtin_bit_cast(bf16x8, make_uint4(u.x, u.y, v.x, v.y));
}
// 16x16x16 product.  For PREC >= 2 the two terms a_hi b_hi + a_lo b_hi go into
// one K = 32 instruction, A = [a_hi | a_lo], B = [b_hi | b_hi] (lane (r, g)
// holds k = 4g..4g+3 of each half, the same k in A and B), which issues at the
// rate of one K = 16 instruction; PREC 3 adds a_hi b_lo as a second K = 32
// instruction with a zero half, so that dependent products never mix the two
// MFMA shapes on one accumulator.
template <int PREC>
__device__ __forceinline__ f32x4 mma4f(const Frag4& a, const Frag4& b, f32x4 c) {
    if constexpr (PREC == 1) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.h, b.h, c, 0, 0, 0);
    } else {
        if constexpr (PREC == 3) {
            const short4v z = short4v{0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cat4(a.h, z), cat4(b.l, z), c, 0, 0, 0);
        }
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(cat4(a.h, a.l), cat4(b.h, b.h), c, 0, 0, 0);
    }
}

__device__ __forceinline__ f32x4 negacc(f32x4 a) { return f32x4{-a[0], -a[1], -a[2], -a[3]}; }

// 16-byte vector of storage elements <-> floats
template <typename ST> struct Vec16;
template <> struct Vec16<uint16_t> {
    static constexpr int N = 8;
    uint4 u;
    __device__ __forceinline__ float get(int i) const {
        const uint32_t w = (i < 2) ? u.x : (i < 4) ? u.y : (i < 6) ? u.z : u.w;
        return (i & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
    }
};
template <> struct Vec16<float> {
    static constexpr int N = 4;
    uint4 u;
    __device__ __forceinline__ float get(int i) const {
        return __uint_as_float((i == 0) ? u.x : (i == 1) ? u.y : (i == 2) ? u.z : u.w);
    }
};

// 16 bytes of storage elements from floats (8 bf16 or 4 fp32)
template <typename ST> __device__ __forceinline__ void store_vec(ST* p, const float* v);
template <> __device__ __forceinline__ void store_vec<uint16_t>(uint16_t* p, const float* v) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack2bf(v[0], v[1]), pack2bf(v[2], v[3]), pack2bf(v[4], v[5]),
                                              pack2bf(v[6], v[7]));
}
template <> __device__ __forceinline__ void store_vec<float>(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// Inclusive prefix sum over the 16 lanes of each DPP row (lanes 16 r .. 16 r +
// 15), in lane order: four row_shr steps, lanes without a source adding 0
__device__ __forceinline__ float row16_scan(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, true));
    return x;
}

// 1 / (1 + e^-x) with the hardware reciprocal (1 ulp); e^-x = inf gives 0
__device__ __forceinline__ float sigm(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// The layer's gated RMSNorm, y = o rsqrt(mean_d o^2 + eps) w sigmoid(z) per
// head of D channels (RMSNormGated, nope_gdn_mlx.py:340-366), on one 16-byte
// piece of a row: o and z hold EPV channels of the row, w their weights; the
// row's other D / EPV - 1 pieces are in the neighbouring lanes (an aligned
// group of consecutive lanes), which must all call this together.
template <typename ST, int D>
__device__ __forceinline__ void gated_rmsnorm_piece(const uint4& o, const uint4& z, const float* w, float eps,
                                                    float* y) {
    constexpr int EPV = 16 / (int)sizeof(ST), VPR = D / EPV;
    static_assert(VPR >= 1 && VPR <= 64 && (VPR & (VPR - 1)) == 0, "row pieces in an aligned lane group");
    const Vec16<ST> ov{o}, zv{z};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPV; ++e) ss = fmaf(ov.get(e), ov.get(e), ss);
#pragma unroll
    for (int m = 1; m < VPR; m <<= 1) ss += __shfl_xor(ss, m, 64);
    const float rs = rsqrtf(ss * (1.f / (float)D) + eps);
#pragma unroll
    for (int e = 0; e < EPV; ++e) y[e] = ov.get(e) * rs * w[e] * sigm(zv.get(e));
}

// ----------------------------------------------------------------------------
// cooperative 16-byte tile copies (256 threads)
// ----------------------------------------------------------------------------
// The prefetched vectors live in one SSA vector value, never in an array: an
// array indexed inside a loop is an alloca that the backend would place in LDS
// or scratch, which forces a wait on every load.
template <typename ST, int ROWS, int COLS, int NTH = 256>
struct Tile {
    static constexpr int EPV = 16 / (int)sizeof(ST);
    static constexpr int VPR = COLS / EPV;
    static constexpr int NV = ROWS * VPR;
    static constexpr int PER = (NV + NTH - 1) / NTH;
    typedef uint32_t vec_t __attribute__((ext_vector_type(4 * PER)));
    vec_t r;
    // bit i: element i lies in a valid row.  Rows past valid_rows are loaded
    // from the last valid row (so the load needs no branch, and the compiler no
    // wait inside one) and read back as zero.
    uint32_t ok = ~0u;

    __device__ __forceinline__ void put(int i, uint4 x) {
        r[4 * i] = x.x; r[4 * i + 1] = x.y; r[4 * i + 2] = x.z; r[4 * i + 3] = x.w;
    }
    __device__ __forceinline__ uint4 get(int i) const {
        const bool v = (ok >> i) & 1u;
        return make_uint4(v ? r[4 * i] : 0u, v ? r[4 * i + 1] : 0u, v ? r[4 * i + 2] : 0u, v ? r[4 * i + 3] : 0u);
    }
    // all ROWS rows are read
    __device__ __forceinline__ void load(const ST* __restrict__ g, size_t gld) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int v = threadIdx.x + NTH * i;
            if (NV % NTH == 0 || v < NV) {
                const int row = v / VPR, c = (v - row * VPR) * EPV;
                put(i, *reinterpret_cast<const uint4*>(g + (size_t)row * gld + c));
            }
        }
    }
    // rows at or past valid_rows (>= 1) read as zero
    __device__ __forceinline__ void load(const ST* __restrict__ g, size_t gld, int valid_rows) {
        load_at(threadIdx.x, g, gld, valid_rows);
    }
    // ... and columns at or past valid_cols (a multiple of EPV, >= EPV) too: a
    // tensor row narrower than the tile, its missing columns zero.  Addresses
    // are clamped into the valid rows and columns.
    __device__ __forceinline__ void load(const ST* __restrict__ g, size_t gld, int valid_rows, int valid_cols) {
        ok = 0u;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int v = threadIdx.x + NTH * i;
            if (NV % NTH == 0 || v < NV) {
                const int row = v / VPR, c = (v - row * VPR) * EPV;
                const int rr = min(row, valid_rows - 1), cc = min(c, valid_cols - EPV);
                put(i, *reinterpret_cast<const uint4*>(g + (size_t)rr * gld + cc));
                ok |= (uint32_t)(row < valid_rows && c < valid_cols) << i;
            }
        }
    }
    __device__ __forceinline__ void store(ST* lds, int lld) const { store_at(threadIdx.x, lds, lld); }

    // the same with an explicit thread index t in [0, 256) (for a 256-thread
    // subset of a larger workgroup)
    __device__ __forceinline__ void load_at(int t, const ST* __restrict__ g, size_t gld) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int v = t + NTH * i;
            if (NV % NTH == 0 || v < NV) {
                const int row = v / VPR, c = (v - row * VPR) * EPV;
                put(i, *reinterpret_cast<const uint4*>(g + (size_t)row * gld + c));
            }
        }
    }
    __device__ __forceinline__ void load_at(int t, const ST* __restrict__ g, size_t gld, int valid_rows) {
        ok = 0u;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int v = t + NTH * i;
            if (NV % NTH == 0 || v < NV) {
                const int row = v / VPR, c = (v - row * VPR) * EPV;
                const int rr = min(row, valid_rows - 1);
                put(i, *reinterpret_cast<const uint4*>(g + (size_t)rr * gld + c));
                ok |= (uint32_t)(row < valid_rows) << i;
            }
        }
    }
    __device__ __forceinline__ void store_at(int t, ST* lds, int lld) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int v = t + NTH * i;
            if (NV % NTH == 0 || v < NV) {
                const int row = v / VPR, c = (v - row * VPR) * EPV;
                *reinterpret_cast<uint4*>(lds + row * lld + c) = get(i);
            }
        }
    }
};

template <typename ST, int ROWS, int COLS>
__device__ __forceinline__ void tile_out_at(int t, const ST* lds, int lld, ST* __restrict__ g, size_t gld,
                                            int valid_rows) {
    constexpr int EPV = 16 / (int)sizeof(ST), VPR = COLS / EPV, NV = ROWS * VPR;
    for (int v = t; v < NV; v += 256) {
        const int row = v / VPR, c = (v - row * VPR) * EPV;
        if (row < valid_rows)
            *reinterpret_cast<uint4*>(g + (size_t)row * gld + c) = *reinterpret_cast<const uint4*>(lds + row * lld + c);
    }
}

template <typename ST, int ROWS, int COLS, int NTH = 256>
__device__ __forceinline__ void tile_out(const ST* lds, int lld, ST* __restrict__ g, size_t gld, int valid_rows) {
    constexpr int EPV = 16 / (int)sizeof(ST), VPR = COLS / EPV, NV = ROWS * VPR, PER = (NV + NTH - 1) / NTH;
    // a fixed number of unrolled steps (no loop with a data-dependent count), so
    // the compiler can count the stores in flight exactly
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int v = (int)threadIdx.x + NTH * i;
        const int row = v / VPR, c = (v - row * VPR) * EPV;
        if (v < NV && row < valid_rows)
            *reinterpret_cast<uint4*>(g + (size_t)row * gld + c) = *reinterpret_cast<const uint4*>(lds + row * lld + c);
    }
}

// tile_out for a [ROWS][D] output tile with the gated RMSNorm fused: each row
// is stored as o and as y = gated_rmsnorm(o, z) (gated_rmsnorm_piece).  The
// VPR = D / EPV threads of a row are consecutive lanes; z rows past
// valid_rows are clamped (read, not used), so every lane reaches the shuffles.
template <typename ST, int ROWS, int D, int NTH = 256>
__device__ __forceinline__ void tile_out_gated(int t, const ST* lds, int lld, ST* __restrict__ go, size_t gld,
                                               ST* __restrict__ gy, size_t ld_y, const ST* __restrict__ gz,
                                               size_t ld_z, const float* __restrict__ nw, float eps,
                                               int valid_rows) {
    constexpr int EPV = 16 / (int)sizeof(ST), VPR = D / EPV, NV = ROWS * VPR;
    static_assert(NV % NTH == 0 && NTH % VPR == 0, "whole rows per pass");
    const int c = (t % VPR) * EPV;
    float w[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) w[e] = nw[c + e];
#pragma unroll
    for (int i = 0; i < NV / NTH; ++i) {
        const int row = (t + NTH * i) / VPR, rz = min(row, valid_rows - 1);
        const uint4 ov = *reinterpret_cast<const uint4*>(lds + row * lld + c);
        const uint4 zv = *reinterpret_cast<const uint4*>(gz + (size_t)rz * ld_z + c);
        float y[EPV];
        gated_rmsnorm_piece<ST, D>(ov, zv, w, eps, y);
        if (row < valid_rows) {
            *reinterpret_cast<uint4*>(go + (size_t)row * gld + c) = ov;
            store_vec<ST>(gy + (size_t)row * ld_y + c, y);
        }
    }
}

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

// ----------------------------------------------------------------------------
// LDS DMA (gfx950 global_load_lds_dwordx4): one wave instruction moves 64 x 16
// bytes from per-lane global addresses into 1 KB of LDS, lane l landing at
// base + 16 l, without passing through registers.  Completion is counted by
// vmcnt; a workgroup fence would wait for all of them, so kernels that keep
// DMA in flight across barriers use lds_barrier() and dma_wait<N>() instead of
// __syncthreads().
// ----------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

// Issued as inline assembly with the LDS base bound to M0.  The compiler's
// wait-count pass does not see it, so it cannot conservatively drain every DMA
// in flight before an unrelated LDS access (which it does for the builtin
// whenever it cannot tell the DMA target and the access apart).  Callers wait
// for their DMA explicitly with dma_wait<N>() before the barrier that
// publishes it; compiler-generated vmcnt waits for other memory operations
// stay correct, only more conservative, because a DMA issued after such an
// operation completes after it.  The s_nop covers the M0-write -> LDS-DMA
// hazard that the compiler's hazard recognizer does not see through asm.
__device__ __forceinline__ void dma16(const void* g, void* lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds_base);
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m) : "memory");
}

// the same with a wave-uniform 64-bit base (SGPRs) and a 32-bit per-lane offset
__device__ __forceinline__ void dma16_s(const void* gbase, uint32_t off, void* lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds_base);
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(gbase), "{m0}"(m) : "memory");
}

// 32-bit LDS address of a (non-null) shared-memory pointer, computed once so
// that each DMA only adds a constant to it
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    __builtin_assume(p != nullptr);
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void_t*)p);
}
// dma16_s with the LDS destination as a 32-bit address (wave-uniform)
__device__ __forceinline__ void dma16_s32(const void* gbase, uint32_t off, uint32_t m) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(gbase), "{m0}"(m) : "memory");
}

// one 4-byte LDS DMA per active lane (lane l lands at m + 4 l): used to pull
// whole cache lines into L2 ahead of their use, the LDS bytes being scratch
__device__ __forceinline__ void dma4(const void* g, uint32_t m) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(m) : "memory");
}

// s_waitcnt immediates (gfx9 layout: vmcnt [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
template <int N>
__device__ __forceinline__ void dma_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// vmcnt wait: all but the last `k` chunks' DMA (L instructions each) complete
template <int L>
__device__ __forceinline__ void dma_wait_chunks(int k) {
    if (k >= 2) dma_wait<2 * L>();
    else if (k == 1) dma_wait<L>();
    else dma_wait<0>();
}

// This wave's LDS writes complete, then the workgroup barrier.  The empty asm
// statements keep the compiler from moving memory operations across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Swizzled LDS tiles: rows of RB bytes (a multiple of 16); the 16-byte chunk c
// of row r is stored at chunk c ^ (r & M), M = min(RB / 16, 8) - 1, so that
// the 16 rows an MFMA fragment read touches spread over the banks.
template <int RB>
struct Swz {
    static constexpr int NCH = RB / 16, M = (NCH < 8 ? NCH : 8) - 1;
    // byte offset of byte b of row r
    __device__ __forceinline__ static int at(int r, int b) { return r * RB + ((((b >> 4) ^ (r & M))) << 4) + (b & 15); }
};

// Fill an NR x RB-byte swizzled LDS tile from a global tile whose rows are GS
// bytes apart.  The tile is NR * RB / 1024 wave-instructions; wave `first` of
// STEP waves issues instructions first, first + STEP, ... (COUNT of them), lane
// l of instruction i filling LDS bytes [1024 i + 16 l, +16).  Rows at or past
// valid_rows are not loaded (their lanes are inactive).
template <int NR, int RB, int STEP>
struct DmaTile {
    static constexpr int NI = NR * RB / 1024, COUNT = NI / STEP;
    static_assert((NR * RB) % 1024 == 0 && NI % STEP == 0, "tile must split into whole 1 KB blocks per wave");
    // per-lane byte offsets of this wave's instructions (fixed for a kernel)
    __device__ __forceinline__ static void offsets(uint32_t (&off)[COUNT], size_t GS, int first, int lane) {
#pragma unroll
        for (int k = 0; k < COUNT; ++k) {
            const int i = first + STEP * k;
            const int p = 1024 * i + 16 * lane, r = p / RB, pc = (p % RB) >> 4;
            off[k] = (uint32_t)(r * GS) + ((uint32_t)(pc ^ (r & Swz<RB>::M)) << 4);
        }
    }
    // all rows valid: wave-uniform base plus the precomputed offsets
    __device__ __forceinline__ static void issue_s(const char* g, const uint32_t (&off)[COUNT], char* lds, int first) {
#pragma unroll
        for (int k = 0; k < COUNT; ++k) dma16_s(g, off[k], lds + 1024 * (first + STEP * k));
    }
    // the same with the destination as a 32-bit LDS address
    __device__ __forceinline__ static void issue_s32(const char* g, const uint32_t (&off)[COUNT], uint32_t lds,
                                                     int first) {
#pragma unroll
        for (int k = 0; k < COUNT; ++k) dma16_s32(g, off[k], lds + 1024 * (first + STEP * k));
    }
    __device__ __forceinline__ static void issue(const char* g, size_t GS, char* lds, int first, int lane,
                                                 int valid_rows = NR) {
#pragma unroll
        for (int k = 0; k < COUNT; ++k) {
            const int i = first + STEP * k;
            const int p = 1024 * i + 16 * lane, r = p / RB, pc = (p % RB) >> 4;
            const int c = pc ^ (r & Swz<RB>::M);
            if (r < valid_rows) dma16(g + (size_t)r * GS + (c << 4), lds + 1024 * i);
        }
    }
};

// MFMA fragment (16x16x32 bf16, same k-slot order as ldfrag) from a swizzled
// bf16 tile with RB-byte rows: rows row0 + l%16, k = k0 + 4 (l/16) + {0..3, 16..19}
template <int RB>
__device__ __forceinline__ Frag8 ldfrag_sw(const uint16_t* M, int row0, int k0) {
    const int l = lane_id(), r = row0 + (l & 15), g = l >> 4;
    const char* base = reinterpret_cast<const char*>(M);
    const uint2 x = *reinterpret_cast<const uint2*>(base + Swz<RB>::at(r, 2 * (k0 + 4 * g)));
    const uint2 y = *reinterpret_cast<const uint2*>(base + Swz<RB>::at(r, 2 * (k0 + 4 * g + 16)));
    Frag8 f;
    f.h = __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
    return f;
}
// ldfragT on a swizzled tile: the A (or B) fragment whose row (n) index runs
// along the tile's columns n0.. and whose k index along its rows k0..  Each
// lane's 8-byte piece lies inside one 16-byte chunk, which the swizzle keeps
// whole.
template <int RB>
__device__ __forceinline__ Frag8 ldfragT_sw(const uint16_t* M, int n0, int k0) {
    const int l = lane_id(), j = l & 15, g = l >> 4, r = k0 + 4 * g + (j >> 2), b = 2 * (n0 + 4 * (j & 3));
    const char* base = reinterpret_cast<const char*>(M);
    const short4v x = ld_tr4(reinterpret_cast<const uint16_t*>(base + Swz<RB>::at(r, b)));
    const short4v y = ld_tr4(reinterpret_cast<const uint16_t*>(base + Swz<RB>::at(r + 16, b)));
    Frag8 f;
    f.h = __builtin_bit_cast(bf16x8, short8v{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]});
    return f;
}
// ld_col4 on a swizzled tile: rows k0 + 4 g + e of column n0 + (l % 16), the
// accumulator layout of a 16-row block
template <int RB>
__device__ __forceinline__ f32x4 ld_col4_sw(const uint16_t* M, int n0, int k0) {
    const int l = lane_id(), j = l & 15, g = l >> 4;
    const short4v x = ld_tr4(reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(M) +
                                                                Swz<RB>::at(k0 + 4 * g + (j >> 2), 2 * (n0 + 4 * (j & 3)))));
    return f32x4{bf2f((uint16_t)x[0]), bf2f((uint16_t)x[1]), bf2f((uint16_t)x[2]), bf2f((uint16_t)x[3])};
}

// one bf16 element (row r, column c) of a swizzled tile, as float
template <int RB>
__device__ __forceinline__ float ld_sw(const uint16_t* M, int r, int c) {
    return bf2f(*reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(M) + Swz<RB>::at(r, 2 * c)));
}

}  // namespace kda
