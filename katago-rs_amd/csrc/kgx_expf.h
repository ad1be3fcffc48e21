// The constants of glibc's expf (the reference calls its port of it: crates/katago-core/src/port/math.rs:634-680),
// shared by the device's post-processing (kgx_post.hip) and the check of the restatement against the host's expf
// (tests/expf_check.cpp). exp(x) = 2^(k/32) 2^(r/32) with x 32/ln 2 = k + r: entry i of the table is the bits of the
// double nearest 2^(i/32) minus i 2^47 (so that adding k 2^47 puts k / 32 into the exponent), and 2^(r/32) is the
// cubic 1 + C2 r + C1 r^2 + C0 r^3 with the minimax coefficients of ARM's optimized-routines expf, scaled by 1/32.
#pragma once

constexpr unsigned long long kgx_exp2f_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};
constexpr double kgx_exp2f_invln2n = 0x1.71547652b82fep+5;  // 32 / ln 2
constexpr double kgx_exp2f_shift = 0x1.8p+52;
constexpr double kgx_exp2f_c0 = 0x1.c6af84b912394p-5 / 32768.0, kgx_exp2f_c1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 kgx_exp2f_c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
