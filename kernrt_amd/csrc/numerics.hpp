// Scalar numerics shared by the HIP kernels and the host side of the backend.
//
// Every function here is bit-for-bit the arithmetic of the reference KernRT
// CPU path on x86-64 Linux, so the device can reproduce its results exactly:
//  * f16 scale encoding/decoding of the Q8_0 block format (quant.rs:722-769),
//  * the int8 rounding rule of the quantizers (quant.rs:843, 871),
//  * `f32::exp`, which Rust lowers to glibc's `expf`. glibc >= 2.28 uses the
//    published ARM optimized-routines method (MIT / Apache-2.0): a 32-entry
//    2^(i/32) table and a degree-3 polynomial evaluated in double. On x86-64
//    CPUs with FMA (any host of an MI355X) glibc selects its FMA build, whose
//    contractions are reproduced below. This restatement was checked equal to
//    glibc 2.35 `expf` on all 2^32 inputs (tests/test_numerics.py samples it
//    and runs the exhaustive sweep under KERNRT_SLOW=1).
//
// Compile with -ffp-contract=off: only the explicit fma() calls may fuse.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define KR_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#define KR_HD static inline
#endif

namespace kr {

KR_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
KR_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
KR_HD uint64_t d2u(double f) { return __builtin_bit_cast(uint64_t, f); }
KR_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// Round-to-nearest-even f32 -> IEEE binary16 bits, integer-only (quant.rs:722-758).
KR_HD uint16_t f32_to_f16_bits(float value) {
    uint32_t bits = f2u(value);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exp = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = bits & 0x007fffffu;
    if (((bits >> 23) & 0xffu) == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant != 0 ? 0x0200u : 0u));
    if (exp <= 0) {
        if (exp < -10) return (uint16_t)sign;
        uint32_t significand = mant | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - exp);
        uint32_t base = significand >> shift;
        uint32_t rem = significand & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        uint32_t up = (rem > halfway || (rem == halfway && (base & 1u) != 0u)) ? 1u : 0u;
        return (uint16_t)(sign | (base + up));
    }
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    uint32_t base = mant >> 13;
    uint32_t rem = mant & 0x1fffu;
    uint32_t rounded = base + ((rem > 0x1000u || (rem == 0x1000u && (base & 1u) != 0u)) ? 1u : 0u);
    int32_t e = exp;
    if (rounded == 0x400u) {
        e += 1;
        rounded = 0;
    }
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | rounded);
}

// The reference's normal-only f16 widening (quant.rs:764-769). A code with a
// zero exponent field widens to 2^-15 * (1 + m/1024), not to zero/subnormal,
// which is why a hardware f16->f32 convert cannot be used here.
// sign | ((exp + 112) << 23) | (mant << 13), as two masks, a shift-add and
// a shift-or: the exponent and mantissa move up 13 bits together and the
// rebase by 112 is one add (exp + 112 <= 143 never reaches the sign bit).
KR_HD float f16w(uint16_t bits) {
    const uint32_t h = bits;
    return u2f(((h & 0x8000u) << 16) | (((h & 0x7fffu) << 13) + (112u << 23)));
}

// `(t).round().clamp(-127.0, 127.0) as i8` (quant.rs:843): round half away
// from zero, clamp, saturating cast with NaN -> 0.
KR_HD int8_t q8_round(float t) {
    float r = __builtin_roundf(t);
    if (r != r) return 0;
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int32_t)r;
}

// total_cmp key (generate.rs:70-77 uses Iterator::max_by(total_cmp)).
KR_HD int32_t total_order_key(float f) {
    int32_t k = (int32_t)f2u(f);
    k ^= (int32_t)(((uint32_t)(k >> 31)) >> 1);
    return k;
}

// glibc expf (see the header comment). T[i] = bits(2^(i/32)) - (i << 47).
#if defined(__HIP_DEVICE_COMPILE__)
__device__ __constant__ static const uint64_t kExp2Tab[32] = {
#else
static const uint64_t kExp2Tab[32] = {
#endif
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// `tab` holds kExp2Tab; a kernel may pass a copy in LDS.
KR_HD float glibc_expf(float x, const uint64_t* tab) {
    const double N = 32.0;
    const double InvLn2N = 0x1.71547652b82fep+0 * N;
    const double Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double C1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double C2 = 0x1.62e42ff0c52d6p-1 / N;
    uint32_t ux = f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 or x is nan
        if (ux == 0xff800000u) return 0.0f;           // -inf
        if (abstop >= 0x7f8u) return x + x;           // +inf or nan
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;          // underflow
    }
    double xd = (double)x;
    double z = InvLn2N * xd;
    double kd = z + Shift;
    uint64_t ki = d2u(kd);
    kd -= Shift;
    double r = __builtin_fma(InvLn2N, xd, -kd);
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s = u2d(t);
    double p = __builtin_fma(C0, r, C1);
    double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}

KR_HD float glibc_expf(float x) { return glibc_expf(x, kExp2Tab); }

}  // namespace kr
