// Scalar helpers shared by the kernels: correctly rounded arithmetic in the
// input type, the reference's public predicate, and small vector types.
#pragma once

#include "nl_device.h"

#include <cmath>

namespace tnr {

template <typename T>
struct Ops;

template <>
struct Ops<float> {
    static constexpr double eps = 1.1920928955078125e-07;
    static constexpr double max = 3.4028234663852886e+38;
    __device__ static float add(float a, float b) { return __fadd_rn(a, b); }
    __device__ static float sub(float a, float b) { return __fsub_rn(a, b); }
    __device__ static float mul(float a, float b) { return __fmul_rn(a, b); }
    __device__ static float fma_(float a, float b, float c) { return __fmaf_rn(a, b, c); }
    // Correctly rounded, in every kernel: HIP's __fsqrt_rn is the native
    // square root (about 1 ulp) unless OCML_BASIC_ROUNDED_OPERATIONS is
    // defined, and the optimiser may or may not drop its accuracy note; a
    // plain llvm.sqrt.f32 (HIP's default correctly rounded divide / sqrt)
    // is lowered to the correctly rounded sequence.
    __device__ static float sqrt_(float a) { return __builtin_sqrtf(a); }
    // Nearest float not below / not above x.
    __device__ static float down(double x) {
        float f = (float)x;
        if ((double)f > x) f = nextafterf(f, -INFINITY);
        return f;
    }
    __device__ static float up(double x) {
        float f = (float)x;
        if ((double)f < x) f = nextafterf(f, INFINITY);
        return f;
    }
};

template <>
struct Ops<double> {
    static constexpr double eps = 2.220446049250313e-16;
    static constexpr double max = 1.7976931348623157e+308;
    __device__ static double add(double a, double b) { return __dadd_rn(a, b); }
    __device__ static double sub(double a, double b) { return __dsub_rn(a, b); }
    __device__ static double mul(double a, double b) { return __dmul_rn(a, b); }
    __device__ static double fma_(double a, double b, double c) { return __fma_rn(a, b, c); }
    __device__ static double sqrt_(double a) { return __dsqrt_rn(a); }
    __device__ static double down(double x) { return x; }
    __device__ static double up(double x) { return x; }
};

template <typename T>
struct alignas(4 * sizeof(T)) Vec4 {
    T x, y, z, w;
};

// The atom index rides in the fourth lane of a binned record.
__device__ __forceinline__ float idx_as(int i, float) { return __int_as_float(i); }
__device__ __forceinline__ double idx_as(int i, double) { return (double)i; }
__device__ __forceinline__ int as_idx(float v) { return __float_as_int(v); }
__device__ __forceinline__ int as_idx(double v) { return (int)v; }

// Status word as left by the earlier kernels of the request: a plain load
// (a kernel boundary makes their writes visible; bits raised meanwhile by
// other workgroups of the running kernel may or may not be seen).
__device__ __forceinline__ unsigned long long load_status(const unsigned long long* s) {
    return *s;
}

__device__ __forceinline__ int floor_div(int a, int b) {
    int q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
}

// The public predicate of the reference (neighbors_cpu.cpp:247-261): D =
// (p_t - p_s) + S0 c0 + S1 c1 + S2 c2 with every product and sum rounded in
// T in this order, d2 = D0^2 + D1^2 + D2^2 left to right.  Writes D, returns d2.
template <typename T, typename I>
__device__ __forceinline__ T public_vector(const T ps[3], const T pt[3], I S0, I S1, I S2,
                                           const T* cell, T D[3]) {
    using O = Ops<T>;
    const T s0 = (T)S0, s1 = (T)S1, s2 = (T)S2;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        T comp = O::sub(pt[c], ps[c]);
        comp = O::add(comp, O::mul(s0, cell[c]));
        comp = O::add(comp, O::mul(s1, cell[3 + c]));
        comp = O::add(comp, O::mul(s2, cell[6 + c]));
        D[c] = comp;
    }
    T d2 = O::mul(D[0], D[0]);
    d2 = O::add(d2, O::mul(D[1], D[1]));
    d2 = O::add(d2, O::mul(D[2], D[2]));
    return d2;
}

// Same value for a cell whose off-diagonal entries are all zero: the skipped
// products are signed zeros, whose addition leaves every nonzero sum
// unchanged, so D equals the general formula (up to the sign of a zero).
template <typename T, typename I>
__device__ __forceinline__ T public_vector_diag(const T ps[3], const T pt[3], I S0, I S1, I S2,
                                                const T* cell, T D[3]) {
    using O = Ops<T>;
    D[0] = O::add(O::sub(pt[0], ps[0]), O::mul((T)S0, cell[0]));
    D[1] = O::add(O::sub(pt[1], ps[1]), O::mul((T)S1, cell[4]));
    D[2] = O::add(O::sub(pt[2], ps[2]), O::mul((T)S2, cell[8]));
    T d2 = O::mul(D[0], D[0]);
    d2 = O::add(d2, O::mul(D[1], D[1]));
    d2 = O::add(d2, O::mul(D[2], D[2]));
    return d2;
}

__device__ __forceinline__ bool fits_i32(long long v) {
    return v >= -2147483648ll && v <= 2147483647ll;
}

// The same for an integer held exactly in a double.
__device__ __forceinline__ bool fits_i32d(double v) {
    return v >= -2147483648.0 && v <= 2147483647.0;
}

// ----------------------------------------------------------- wave reductions

__device__ __forceinline__ long long wave_inclusive_scan(long long x) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const long long y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

// Inclusive wave64 scans of 32-bit values with DPP lane moves (no LDS
// crossbar): four row shifts build 16-lane row prefixes, then row_bcast:15
// carries row 0 into row 1 and row 2 into row 3, and row_bcast:31 carries
// rows 0-1 into rows 2-3.  Lanes whose source lane is outside the row (or
// whose row is masked off) read the identity 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_move(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, false);
}

__device__ __forceinline__ int wave_inclusive_scan_i32(int x) {
    x += dpp_move<0x111, 0xf>(x);  // row_shr:1
    x += dpp_move<0x112, 0xf>(x);  // row_shr:2
    x += dpp_move<0x114, 0xf>(x);  // row_shr:4
    x += dpp_move<0x118, 0xf>(x);  // row_shr:8
    x += dpp_move<0x142, 0xa>(x);  // row_bcast:15 into rows 1, 3
    x += dpp_move<0x143, 0xc>(x);  // row_bcast:31 into rows 2, 3
    return x;
}

// Inclusive running maximum of non-negative values.
__device__ __forceinline__ int wave_inclusive_max_i32(int x) {
    x = max(x, dpp_move<0x111, 0xf>(x));
    x = max(x, dpp_move<0x112, 0xf>(x));
    x = max(x, dpp_move<0x114, 0xf>(x));
    x = max(x, dpp_move<0x118, 0xf>(x));
    x = max(x, dpp_move<0x142, 0xa>(x));
    x = max(x, dpp_move<0x143, 0xc>(x));
    return x;
}

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long x) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        const unsigned long long y = __shfl_xor(x, d);
        x = y < x ? y : x;
    }
    return x;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        const unsigned long long y = __shfl_xor(x, d);
        x = y > x ? y : x;
    }
    return x;
}

// Unsigned maximum over the wave, every lane receives it (DPP row shifts
// and broadcasts; lanes whose source is outside the row read 0, the
// identity).
__device__ __forceinline__ unsigned wave_max_u32(unsigned x) {
    x = max(x, (unsigned)dpp_move<0x111, 0xf>((int)x));
    x = max(x, (unsigned)dpp_move<0x112, 0xf>((int)x));
    x = max(x, (unsigned)dpp_move<0x114, 0xf>((int)x));
    x = max(x, (unsigned)dpp_move<0x118, 0xf>((int)x));
    x = max(x, (unsigned)dpp_move<0x142, 0xa>((int)x));
    x = max(x, (unsigned)dpp_move<0x143, 0xc>((int)x));
    return (unsigned)__builtin_amdgcn_readlane((int)x, kWave - 1);
}

// Maximum of x over the lanes [head, lane] of a contiguous segment that
// starts at lane `head` (segmented inclusive scan with lane shuffles).
__device__ __forceinline__ unsigned long long segment_max_u64(unsigned long long x, int head) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const unsigned long long y = __shfl_up(x, d);
        if (lane - d >= head) x = y > x ? y : x;
    }
    return x;
}

// ------------------------------------------------- reduction key encodings
// Max-keys of the atom reductions (see RedSlot): 32-bit keys for float
// inputs, 64-bit for double.  ord32 / order_key map numeric order to
// unsigned order.
__device__ __forceinline__ unsigned ord32(float x) {
    const unsigned b = __float_as_uint(x);
    return (b >> 31) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float ord32_value(unsigned k) {
    const unsigned b = (k >> 31) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

template <typename T>
struct RedKeys;

template <>
struct RedKeys<float> {
    // bounds rounded outward to float: the bins still cover every atom
    __device__ static unsigned long long lower(double x) { return (unsigned long long)~ord32(Ops<float>::down(x)); }
    __device__ static unsigned long long upper(double x) { return ord32(Ops<float>::up(x)); }
    __device__ static unsigned long long lower_exact(float x) { return (unsigned long long)~ord32(x); }
    __device__ static unsigned long long upper_exact(float x) { return ord32(x); }
    // non-negative, rounded up: only enlarges the margin
    __device__ static unsigned long long magnitude(double x) { return __float_as_uint(Ops<float>::up(x)); }
    __device__ static double lower_value(unsigned long long k) { return (double)ord32_value(~(unsigned)k); }
    __device__ static double upper_value(unsigned long long k) { return (double)ord32_value((unsigned)k); }
    __device__ static double magnitude_value(unsigned long long k) { return (double)__uint_as_float((unsigned)k); }
    __device__ static unsigned long long wave_max(unsigned long long x) { return wave_max_u32((unsigned)x); }
};

template <>
struct RedKeys<double> {
    __device__ static unsigned long long lower(double x) { return ~order_key(x); }
    __device__ static unsigned long long upper(double x) { return order_key(x); }
    __device__ static unsigned long long lower_exact(double x) { return ~order_key(x); }
    __device__ static unsigned long long upper_exact(double x) { return order_key(x); }
    __device__ static unsigned long long magnitude(double x) { return (unsigned long long)__double_as_longlong(x); }
    __device__ static double lower_value(unsigned long long k) { return key_value(~k); }
    __device__ static double upper_value(unsigned long long k) { return key_value(k); }
    __device__ static double magnitude_value(unsigned long long k) { return __longlong_as_double((long long)k); }
    __device__ static unsigned long long wave_max(unsigned long long x) { return wave_max_u64(x); }
};

// ------------------------------------------- x87 extended precision, emulated
// The reference evaluates its cell-list padding in long double, the x87
// 80-bit format of its x86-64 builds: a 64-bit significand, every operation
// rounded to nearest even.  Ext holds such a value exactly as an unevaluated
// sum hi + lo of two doubles (hi the double nearest the value), for the
// finite, normal magnitudes of that computation.  Sums are formed exactly
// (two_sum) before the rounding to 64 bits; a sum of two values whose
// exponents lie more than about 40 apart is rounded from a 106-bit
// approximation, which differs from the x87 result only when the exact sum
// lies within 2^-106 of a rounding boundary.
struct Ext {
    double hi, lo;
};

__device__ __forceinline__ Ext two_sum(double a, double b) {
    const double s = __dadd_rn(a, b);
    const double bb = __dsub_rn(s, a);
    const double e = __dadd_rn(__dsub_rn(a, __dsub_rn(s, bb)), __dsub_rn(b, bb));
    return Ext{s, e};
}

// hi + lo rounded to a 64-bit significand (nearest even); |lo| <= ulp(hi) / 2.
__device__ __forceinline__ Ext ext_round(double hi, double lo) {
    if (lo == 0.0 || hi == 0.0 || !isfinite(hi)) return Ext{hi, lo};
    const unsigned long long bits = (unsigned long long)__double_as_longlong(hi);
    const int e = (int)((bits >> 52) & 0x7ff);
    // spacing of 64-bit significands in hi's binade, halved just below a
    // power of two
    double q = ldexp(1.0, e - 1086);
    if ((bits & 0xfffffffffffffull) == 0 && ((lo < 0) != (hi < 0))) q *= 0.5;
    // lo / q is exact (a power-of-two scaling); rint rounds half to even,
    // and the 64-bit significand's parity is that of the multiple of q
    const double k = rint(lo / q);
    return two_sum(hi, k * q);
}

__device__ __forceinline__ Ext ext_exact(double x) { return Ext{x, 0.0}; }

// a * b rounded to 64 bits (a and b doubles, so the product is exact in Ext).
__device__ __forceinline__ Ext ext_mul(double a, double b) {
    const double p = __dmul_rn(a, b);
    return ext_round(p, __fma_rn(a, b, -p));
}

// a * 2^k, exact.
__device__ __forceinline__ Ext ext_scale(Ext a, int k) { return Ext{ldexp(a.hi, k), ldexp(a.lo, k)}; }

// a + b rounded to 64 bits.
__device__ __forceinline__ Ext ext_add(Ext a, Ext b) {
    const Ext s = two_sum(a.hi, b.hi);
    const Ext t = two_sum(a.lo, b.lo);
    const Ext u = two_sum(s.hi, __dadd_rn(s.lo, t.hi));
    const Ext v = two_sum(u.hi, __dadd_rn(u.lo, t.lo));
    return ext_round(v.hi, v.lo);
}

__device__ __forceinline__ bool ext_less(Ext a, Ext b) {
    return a.hi < b.hi || (a.hi == b.hi && a.lo < b.lo);
}

// The value rounded to nearest even in T (a C++ conversion of a long double).
template <typename T>
__device__ __forceinline__ T ext_to(Ext a);

template <>
__device__ __forceinline__ double ext_to<double>(Ext a) {
    // hi + lo is the exact value: the hardware sum rounds it once
    return __dadd_rn(a.hi, a.lo);
}

template <>
__device__ __forceinline__ float ext_to<float>(Ext a) {
    // hi is the double nearest the value, and every float midpoint is a
    // double: hi rounds as the value does unless hi is a midpoint itself,
    // where the sign of lo decides
    float f = __double2float_rn(a.hi);
    const double df = (double)f;
    if (df != a.hi && a.lo != 0.0) {
        const float g = nextafterf(f, a.hi > df ? INFINITY : -INFINITY);
        const double dg = (double)g;
        if (fabs(dg - a.hi) == fabs(df - a.hi))
            f = (a.lo > 0.0) == (dg > df) ? g : f;
    }
    return f;
}

}  // namespace tnr
