#pragma once
// RoPE rotation of one (a, b) pair by a tabulated angle, shared by every kernel that rotates rows: a*c - b*s and
// a*s + b*c with each product and sum rounded on its own (no FMA), as the reference computes them (ref_ops.cpp:
// 179-181, built with -ffp-contract=off; CMakeLists.txt:72-73). The pragma keeps these products and sums unfused
// whatever contraction mode the including file is compiled with (HIP's default would fuse them into an FMA); it
// covers only operators written here, not helper calls such as __fmul_rn, whose bodies live in HIP's headers.
#include <hip/hip_runtime.h>

__device__ __forceinline__ void rope_rotate(float& a, float& b, float2 cs) {
#pragma clang fp contract(off)
  const float a0 = a, b0 = b;
  a = a0 * cs.x - b0 * cs.y;
  b = a0 * cs.y + b0 * cs.x;
}

// The same rotation returning the pair, for operands that cannot bind to a reference (vector elements).
__device__ __forceinline__ float2 rope_pair(float a, float b, float2 cs) {
  rope_rotate(a, b, cs);
  return make_float2(a, b);
}
