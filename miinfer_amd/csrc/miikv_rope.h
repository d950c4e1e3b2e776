// sin and cos of a RoPE angle, shared by every kernel that rotates keys (the append
// prologue and the fused decode store), so both store the same codes.  Plain C++ with
// a host/device qualifier: the CPU tests compile this same header on the host and
// compare it with the oracle's restatement.
//
// Arithmetic (|a| < 2^17, i.e. positions up to 131072 times step^i <= 1): a
// Cody-Waite reduction by pi/2 in three parts, each subtraction a fused multiply-add
// (one rounding of a - k*P_i, so the exactness of k*P1 itself does not matter), then
// the Taylor polynomials of sin and cos on [-pi/4, pi/4] (truncation below 1e-11) in
// Horner form, and the quadrant.  Within 2.5 float32 ulps of float64 sin and cos where
// |value| >= 1/16 and 1e-7 absolute elsewhere.  No contraction beyond the fmaf calls
// written here: every other product and sum rounds as written.
#pragma once

#ifdef __HIPCC__
#define MIIKV_HD __host__ __device__
#else
#define MIIKV_HD
#endif

#include <math.h>

namespace miikv {

MIIKV_HD inline void rope_sincos(float a, float* s, float* c) {
#pragma clang fp contract(off)
    const float k = rintf(a * 6.366197467e-01f);
    float r = fmaf(-k, 1.5703125f, a);
    r = fmaf(-k, 4.838267923e-04f, r);
    r = fmaf(-k, 2.563282919e-12f, r);
    const float r2 = r * r;
    float ps = fmaf(r2, -2.505210794e-08f, 2.755731884e-06f);
    ps = fmaf(r2, ps, -1.984127011e-04f);
    ps = fmaf(r2, ps, 8.333333768e-03f);
    ps = fmaf(r2, ps, -1.666666716e-01f);
    const float sr = fmaf(r * r2, ps, r);
    float pc = fmaf(r2, 2.087675588e-09f, -2.755731998e-07f);
    pc = fmaf(r2, pc, 2.480158764e-05f);
    pc = fmaf(r2, pc, -1.388888923e-03f);
    pc = fmaf(r2, pc, 4.166666791e-02f);
    pc = fmaf(r2, pc, -5.000000000e-01f);
    const float cr = fmaf(r2, pc, 1.0f);
    const int q = static_cast<int>(k) & 3;
    *s = q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr;
    *c = q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr;
}

}  // namespace miikv
