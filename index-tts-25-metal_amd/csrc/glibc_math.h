// Bit-exact device versions of the glibc 2.35 expf, exp and logf that the reference's
// sampler calls when built for x86-64 (oracle/_ref; the CPU oracle).
//
// The sampler's arithmetic (src/gpt_sampling.cpp) feeds libm results straight into its
// decisions: the float log-softmax of beam search sums expf(v - peak) and takes logf of the
// sum (:207-210), and the top-p and draw probabilities are exp(double(v - max)) (:96, :144).
// A one-ulp difference can move a top-p cut, a draw or a beam score, so these follow glibc's
// own method rather than the device libm:
//   * the ARM optimized-routines algorithms glibc 2.28+ ships (Szabolcs Nagy, 2017-2018):
//     expf: x*N/ln2 = k + r, 2^(k/N) from a 32-entry table, degree-3 polynomial in r, all
//     in double; exp: N = 128 table of 2^(i/N) as scale and relative tail, degree-5
//     polynomial, a separate path for results near the subnormal range; logf: x = 2^k z,
//     z in one of 16 subintervals with a tabulated 1/c and log(c), degree-4 log1p in double;
//   * with the fused multiply-adds of glibc's x86-64 FMA build (the one its ifunc selects on
//     CPUs with FMA, such as the hosts here): every a*b+c that build contracts is an fma()
//     below; every other product and sum is rounded separately (contraction is off here).
// The 2^(i/32) and 2^(i/128) tables are the correctly rounded values (minus the exponent
// bits), the scale's relative tail rounded to double; the polynomial coefficients and the
// logf table are the published constants of those routines.  Checked bit for bit against
// glibc: every float input of expf, every float-valued input of exp and every non-NaN input
// of logf (tests/test_libm_repro.py on the CPU; the device on the GPU in
// tests/test_gpu_libm.py).
//
// Attribution and licence of the restated method.  The structure, polynomial coefficients and
// logf table below follow the ARM optimized-routines implementations of exp, expf and logf:
//   Copyright (c) 2017-2018, Arm Limited.
//   SPDX-License-Identifier: MIT
//   Permission is hereby granted, free of charge, to any person obtaining a copy of this
//   software and associated documentation files (the "Software"), to deal in the Software
//   without restriction, including without limitation the rights to use, copy, modify, merge,
//   publish, distribute, sublicense, and/or sell copies of the Software, and to permit persons
//   to whom the Software is furnished to do so, subject to the following conditions: the above
//   copyright notice and this permission notice shall be included in all copies or substantial
//   portions of the Software.  THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND,
//   EXPRESS OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY, FITNESS
//   FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT.  IN NO EVENT SHALL THE AUTHORS OR COPYRIGHT
//   HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF
//   CONTRACT, TORT OR OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
//   USE OR OTHER DEALINGS IN THE SOFTWARE.
// glibc (2.28 and later) ships the same routines under the LGPL-2.1-or-later with that
// attribution ("Contributed by Szabolcs Nagy, ARM"); the tables of 2^(i/N) here were computed
// from their definition, not taken from either source.
#pragma once
#include <stdint.h>

#if defined(__HIP__)
#define ITTS_HD __host__ __device__
#else
#define ITTS_HD
#endif
// Products and sums below are rounded one by one unless written as fma_d (clang contracts
// a*b+c by default in HIP code; host builds of this header use -ffp-contract=off).
#if defined(__clang__)
#define ITTS_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define ITTS_NO_CONTRACT
#endif

namespace itts {
namespace libm {

ITTS_HD inline uint64_t bits_of(double x) { return __builtin_bit_cast(uint64_t, x); }
ITTS_HD inline double double_of(uint64_t u) { return __builtin_bit_cast(double, u); }
ITTS_HD inline uint32_t bits_of(float x) { return __builtin_bit_cast(uint32_t, x); }
ITTS_HD inline float float_of(uint32_t u) { return __builtin_bit_cast(float, u); }
ITTS_HD inline double fma_d(double a, double b, double c) { return __builtin_fma(a, b, c); }

// ---------------------------------------------------------------- expf
constexpr int kExpfBits = 5;
constexpr int kExpfN = 1 << kExpfBits;
// bits(2^(i/32)) - (i << 47)
constexpr uint64_t kExpfTab[kExpfN] = {
    0x3ff0000000000000, 0x3fefd9b0d3158574, 0x3fefb5586cf9890f, 0x3fef9301d0125b51,
    0x3fef72b83c7d517b, 0x3fef54873168b9aa, 0x3fef387a6e756238, 0x3fef1e9df51fdee1,
    0x3fef06fe0a31b715, 0x3feef1a7373aa9cb, 0x3feedea64c123422, 0x3feece086061892d,
    0x3feebfdad5362a27, 0x3feeb42b569d4f82, 0x3feeab07dd485429, 0x3feea47eb03a5585,
    0x3feea09e667f3bcd, 0x3fee9f75e8ec5f74, 0x3feea11473eb0187, 0x3feea589994cce13,
    0x3feeace5422aa0db, 0x3feeb737b0cdc5e5, 0x3feec49182a3f090, 0x3feed503b23e255d,
    0x3feee89f995ad3ad, 0x3feeff76f2fb5e47, 0x3fef199bdd85529c, 0x3fef3720dcef9069,
    0x3fef5818dcfba487, 0x3fef7c97337b9b5f, 0x3fefa4afa2a490da, 0x3fefd0765b6e4540,
};

ITTS_HD inline float expf_glibc(float x) {
    ITTS_NO_CONTRACT
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kExpfN, kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / kExpfN / kExpfN / kExpfN, kC1 = 0x1.ebfce50fac4f3p-3 / kExpfN / kExpfN,
                     kC2 = 0x1.62e42ff0c52d6p-1 / kExpfN;
    const uint32_t abstop = (bits_of(x) >> 20) & 0x7ff;
    if (abstop >= (bits_of(88.0f) >> 20)) {  // |x| >= 88, inf or nan
        if (bits_of(x) == bits_of(-__builtin_inff())) return 0.0f;
        if (abstop >= (bits_of(__builtin_inff()) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = x;
    double kd = fma_d(kInvLn2N, xd, kShift);  // round(x N / ln2) in the low bits
    const uint64_t ki = bits_of(kd);
    kd -= kShift;
    const double r = fma_d(kInvLn2N, xd, -kd);
    const double s = double_of(kExpfTab[ki % kExpfN] + (ki << (52 - kExpfBits)));
    const double z = fma_d(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma_d(kC2, r, 1.0);
    y = fma_d(z, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

// ---------------------------------------------------------------- exp
constexpr int kExpBits = 7;
constexpr int kExpN = 1 << kExpBits;
// {bits(tail), bits(scale) - (i << 45)}: scale = 2^(i/128) rounded, tail = (2^(i/128) - scale) / scale rounded
constexpr uint64_t kExpTab[2 * kExpN] = {
    0x0000000000000000, 0x3ff0000000000000,
    0x3c9b3b4f1a88bf6e, 0x3feff63da9fb3335,
    0xbc7160139cd8dc5d, 0x3fefec9a3e778061,
    0xbc905e7a108766d1, 0x3fefe315e86e7f85,
    0x3c8cd2523567f613, 0x3fefd9b0d3158574,
    0xbc8bce8023f98efa, 0x3fefd06b29ddf6de,
    0x3c60f74e61e6c861, 0x3fefc74518759bc8,
    0x3c90a3e45b33d399, 0x3fefbe3ecac6f383,
    0x3c979aa65d837b6d, 0x3fefb5586cf9890f,
    0x3c8eb51a92fdeffc, 0x3fefac922b7247f7,
    0x3c3ebe3d702f9cd1, 0x3fefa3ec32d3d1a2,
    0xbc6a033489906e0b, 0x3fef9b66affed31b,
    0xbc9556522a2fbd0e, 0x3fef9301d0125b51,
    0xbc5080ef8c4eea55, 0x3fef8abdc06c31cc,
    0xbc91c923b9d5f416, 0x3fef829aaea92de0,
    0x3c80d3e3e95c55af, 0x3fef7a98c8a58e51,
    0xbc801b15eaa59348, 0x3fef72b83c7d517b,
    0xbc8f1ff055de323d, 0x3fef6af9388c8dea,
    0x3c8b898c3f1353bf, 0x3fef635beb6fcb75,
    0xbc96d99c7611eb26, 0x3fef5be084045cd4,
    0x3c9aecf73e3a2f60, 0x3fef54873168b9aa,
    0xbc8fe782cb86389d, 0x3fef4d5022fcd91d,
    0x3c8a6f4144a6c38d, 0x3fef463b88628cd6,
    0x3c807a05b0e4047d, 0x3fef3f49917ddc96,
    0x3c968efde3a8a894, 0x3fef387a6e756238,
    0x3c875e18f274487d, 0x3fef31ce4fb2a63f,
    0x3c80472b981fe7f2, 0x3fef2b4565e27cdd,
    0xbc96b87b3f71085e, 0x3fef24dfe1f56381,
    0x3c82f7e16d09ab31, 0x3fef1e9df51fdee1,
    0xbc3d219b1a6fbffa, 0x3fef187fd0dad990,
    0x3c8b3782720c0ab4, 0x3fef1285a6e4030b,
    0x3c6e149289cecb8f, 0x3fef0cafa93e2f56,
    0x3c834d754db0abb6, 0x3fef06fe0a31b715,
    0x3c864201e2ac744c, 0x3fef0170fc4cd831,
    0x3c8fdd395dd3f84a, 0x3feefc08b26416ff,
    0xbc86a3803b8e5b04, 0x3feef6c55f929ff1,
    0xbc924aedcc4b5068, 0x3feef1a7373aa9cb,
    0xbc9907f81b512d8e, 0x3feeecae6d05d866,
    0xbc71d1e83e9436d2, 0x3feee7db34e59ff7,
    0xbc991919b3ce1b15, 0x3feee32dc313a8e5,
    0x3c859f48a72a4c6d, 0x3feedea64c123422,
    0xbc9312607a28698a, 0x3feeda4504ac801c,
    0xbc58a78f4817895b, 0x3feed60a21f72e2a,
    0xbc7c2c9b67499a1b, 0x3feed1f5d950a897,
    0x3c4363ed60c2ac11, 0x3feece086061892d,
    0x3c9666093b0664ef, 0x3feeca41ed1d0057,
    0x3c6ecce1daa10379, 0x3feec6a2b5c13cd0,
    0x3c93ff8e3f0f1230, 0x3feec32af0d7d3de,
    0x3c7690cebb7aafb0, 0x3feebfdad5362a27,
    0x3c931dbdeb54e077, 0x3feebcb299fddd0d,
    0xbc8f94340071a38e, 0x3feeb9b2769d2ca7,
    0xbc87deccdc93a349, 0x3feeb6daa2cf6642,
    0xbc78dec6bd0f385f, 0x3feeb42b569d4f82,
    0xbc861246ec7b5cf6, 0x3feeb1a4ca5d920f,
    0x3c93350518fdd78e, 0x3feeaf4736b527da,
    0x3c7b98b72f8a9b05, 0x3feead12d497c7fd,
    0x3c9063e1e21c5409, 0x3feeab07dd485429,
    0x3c34c7855019c6ea, 0x3feea9268a5946b7,
    0x3c9432e62b64c035, 0x3feea76f15ad2148,
    0xbc8ce44a6199769f, 0x3feea5e1b976dc09,
    0xbc8c33c53bef4da8, 0x3feea47eb03a5585,
    0xbc845378892be9ae, 0x3feea34634ccc320,
    0xbc93cedd78565858, 0x3feea23882552225,
    0x3c5710aa807e1964, 0x3feea155d44ca973,
    0xbc93b3efbf5e2228, 0x3feea09e667f3bcd,
    0xbc6a12ad8734b982, 0x3feea012750bdabf,
    0xbc6367efb86da9ee, 0x3fee9fb23c651a2f,
    0xbc80dc3d54e08851, 0x3fee9f7df9519484,
    0xbc781f647e5a3ecf, 0x3fee9f75e8ec5f74,
    0xbc86ee4ac08b7db0, 0x3fee9f9a48a58174,
    0xbc8619321e55e68a, 0x3fee9feb564267c9,
    0x3c909ccb5e09d4d3, 0x3feea0694fde5d3f,
    0xbc7b32dcb94da51d, 0x3feea11473eb0187,
    0x3c94ecfd5467c06b, 0x3feea1ed0130c132,
    0x3c65ebe1abd66c55, 0x3feea2f336cf4e62,
    0xbc88a1c52fb3cf42, 0x3feea427543e1a12,
    0xbc9369b6f13b3734, 0x3feea589994cce13,
    0xbc805e843a19ff1e, 0x3feea71a4623c7ad,
    0xbc94d450d872576e, 0x3feea8d99b4492ed,
    0x3c90ad675b0e8a00, 0x3feeaac7d98a6699,
    0x3c8db72fc1f0eab4, 0x3feeace5422aa0db,
    0xbc65b6609cc5e7ff, 0x3feeaf3216b5448c,
    0x3c7bf68359f35f44, 0x3feeb1ae99157736,
    0xbc93091fa71e3d83, 0x3feeb45b0b91ffc6,
    0xbc5da9b88b6c1e29, 0x3feeb737b0cdc5e5,
    0xbc6c23f97c90b959, 0x3feeba44cbc8520f,
    0xbc92434322f4f9aa, 0x3feebd829fde4e50,
    0xbc85ca6cd7668e4b, 0x3feec0f170ca07ba,
    0x3c71affc2b91ce27, 0x3feec49182a3f090,
    0x3c6dd235e10a73bb, 0x3feec86319e32323,
    0xbc87c50422622263, 0x3feecc667b5de565,
    0x3c8b1c86e3e231d5, 0x3feed09bec4a2d33,
    0xbc91bbd1d3bcbb15, 0x3feed503b23e255d,
    0x3c90cc319cee31d2, 0x3feed99e1330b358,
    0x3c8469846e735ab3, 0x3feede6b5579fdbf,
    0xbc82dfcd978e9db4, 0x3feee36bbfd3f37a,
    0x3c8c1a7792cb3387, 0x3feee89f995ad3ad,
    0xbc907b8f4ad1d9fa, 0x3feeee07298db666,
    0xbc55c3d956dcaeba, 0x3feef3a2b84f15fb,
    0xbc90a40e3da6f640, 0x3feef9728de5593a,
    0xbc68d6f438ad9334, 0x3feeff76f2fb5e47,
    0xbc91eee26b588a35, 0x3fef05b030a1064a,
    0x3c74ffd70a5fddcd, 0x3fef0c1e904bc1d2,
    0xbc91bdfbfa9298ac, 0x3fef12c25bd71e09,
    0x3c736eae30af0cb3, 0x3fef199bdd85529c,
    0x3c8ee3325c9ffd94, 0x3fef20ab5fffd07a,
    0x3c84e08fd10959ac, 0x3fef27f12e57d14b,
    0x3c63cdaf384e1a67, 0x3fef2f6d9406e7b5,
    0x3c676b2c6c921968, 0x3fef3720dcef9069,
    0xbc808a1883ccb5d2, 0x3fef3f0b555dc3fa,
    0xbc8fad5d3ffffa6f, 0x3fef472d4a07897c,
    0xbc900dae3875a949, 0x3fef4f87080d89f2,
    0x3c74a385a63d07a7, 0x3fef5818dcfba487,
    0xbc82919e2040220f, 0x3fef60e316c98398,
    0x3c8e5a50d5c192ac, 0x3fef69e603db3285,
    0x3c843a59ac016b4b, 0x3fef7321f301b460,
    0xbc82d52107b43e1f, 0x3fef7c97337b9b5f,
    0xbc892ab93b470dc9, 0x3fef864614f5a129,
    0x3c74b604603a88d3, 0x3fef902ee78b3ff6,
    0x3c83c5ec519d7271, 0x3fef9a51fbc74c83,
    0xbc8ff7128fd391f0, 0x3fefa4afa2a490da,
    0xbc8dae98e223747d, 0x3fefaf482d8e67f1,
    0x3c8ec3bc41aa2008, 0x3fefba1bee615a27,
    0x3c842b94c3a9eb32, 0x3fefc52b376bba97,
    0x3c8a64a931d185ee, 0x3fefd0765b6e4540,
    0xbc8e37bae43be3ed, 0x3fefdbfdad9cbe14,
    0x3c77893b4d91cd9d, 0x3fefe7c1819e90d8,
    0x3c5305c14160cc89, 0x3feff3c22b8f71f1,
};

ITTS_HD inline double exp_special(double tmp, uint64_t sbits, uint64_t ki) {
    ITTS_NO_CONTRACT
    if ((ki & 0x80000000) == 0) {  // k > 0: the scale's exponent may have overflowed
        sbits -= 1009ull << 52;
        const double scale = double_of(sbits);
        return 0x1p1009 * fma_d(scale, tmp, scale);
    }
    sbits += 1022ull << 52;  // k < 0: results near the subnormal range
    const double scale = double_of(sbits);
    const double st = scale * tmp;
    double y = scale + st;
    if (y < 1.0) {
        double lo = scale - y + st;
        const double hi = 1.0 + y;
        lo = 1.0 - hi + y + lo;
        y = (hi + lo) - 1.0;
        if (y == 0.0) y = 0.0;
    }
    return 0x1p-1022 * y;
}

ITTS_HD inline double exp_glibc(double x) {
    ITTS_NO_CONTRACT
    constexpr double kInvLn2N = 0x1.71547652b82fep0 * kExpN, kShift = 0x1.8p52;
    constexpr double kNegLn2HiN = -0x1.62e42fefa0000p-8, kNegLn2LoN = -0x1.cf79abc9e3b3ap-47;
    constexpr double kC2 = 0x1.ffffffffffdbdp-2, kC3 = 0x1.555555555543cp-3, kC4 = 0x1.55555cf172b91p-5, kC5 = 0x1.1111167a4d017p-7;
    auto top12 = [](double v) { return static_cast<uint32_t>(bits_of(v) >> 52); };
    uint32_t abstop = top12(x) & 0x7ff;
    if (abstop - top12(0x1p-54) >= top12(512.0) - top12(0x1p-54)) {
        if (abstop - top12(0x1p-54) >= 0x80000000u) return 1.0 + x;  // |x| < 2^-54
        if (abstop >= top12(1024.0)) {
            if (bits_of(x) == bits_of(-__builtin_inf())) return 0.0;
            if (abstop >= top12(__builtin_inf())) return 1.0 + x;
            return (bits_of(x) >> 63) ? 0.0 : __builtin_inf();
        }
        abstop = 0;  // 512 <= |x| < 1024: exp_special
    }
    double kd = fma_d(kInvLn2N, x, kShift);
    const uint64_t ki = bits_of(kd);
    kd -= kShift;
    const double r = fma_d(kd, kNegLn2LoN, fma_d(kd, kNegLn2HiN, x));
    const uint64_t idx = 2 * (ki % kExpN);
    const double tail = double_of(kExpTab[idx]);
    const uint64_t sbits = kExpTab[idx + 1] + (ki << (52 - kExpBits));
    const double r2 = r * r;
    const double tmp = fma_d(r2 * r2, fma_d(r, kC5, kC4), fma_d(r2, fma_d(r, kC3, kC2), tail + r));
    if (abstop == 0) return exp_special(tmp, sbits, ki);
    const double scale = double_of(sbits);
    return fma_d(scale, tmp, scale);
}

// ---------------------------------------------------------------- logf
constexpr int kLogfBits = 4;
constexpr int kLogfN = 1 << kLogfBits;
constexpr double kLogfInvc[kLogfN] = {
    0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0,  0x1.3c995b0b80385p+0,
    0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0,  0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
    0x1.0953f419900a7p+0, 0x1p+0,               0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
    0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1,
};
constexpr double kLogfLogc[kLogfN] = {
    -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
    -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3,   -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611cccp-4,
    -0x1.252f438e10c1ep-5, 0x0p+0,                0x1.aa5aa5df25984p-5,  0x1.c5e53aa362eb4p-4,
    0x1.526e57720db08p-3,  0x1.bc2860d22477p-3,   0x1.1058bc8a07ee1p-2,  0x1.4043057b6ee09p-2,
};

ITTS_HD inline float logf_glibc(float x) {
    ITTS_NO_CONTRACT
    constexpr double kLn2 = 0x1.62e42fefa39efp-1;
    constexpr double kA0 = -0x1.00ea348b88334p-2, kA1 = 0x1.5575b0be00b6ap-2, kA2 = -0x1.ffffef20a4123p-2;
    constexpr uint32_t kOff = 0x3f330000;
    uint32_t ix = bits_of(x);
    if (ix == 0x3f800000) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {  // subnormal, zero, negative, inf, nan
        if (ix * 2 == 0) return -__builtin_inff();
        if (ix == 0x7f800000) return x;
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) return __builtin_nanf("");
        ix = bits_of(x * 0x1p23f);
        ix -= 23u << 23;
    }
    const uint32_t tmp = ix - kOff;
    const int i = static_cast<int>((tmp >> (23 - kLogfBits)) % kLogfN);
    const int k = static_cast<int32_t>(tmp) >> 23;
    const uint32_t iz = ix - (tmp & 0xff800000u);
    const double z = static_cast<double>(float_of(iz));
    const double r = fma_d(z, kLogfInvc[i], -1.0);
    const double y0 = fma_d(static_cast<double>(k), kLn2, kLogfLogc[i]);
    const double r2 = r * r;
    double y = fma_d(kA1, r, kA2);
    y = fma_d(kA0, r2, y);
    y = fma_d(y, r2, y0 + r);
    return static_cast<float>(y);
}

}  // namespace libm
}  // namespace itts
