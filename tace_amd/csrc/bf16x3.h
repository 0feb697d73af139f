// float32 as three bfloat16 terms for the bf16 MFMA.  Each value v is split
// with round-to-nearest-even into v0 = bf16(v), v1 = bf16(v - v0), v2 =
// bf16(v - v0 - v1).  The split is exact, v = v0 + v1 + v2: v - v0 is exact
// in float32 and holds at most 16 significant bits, |v1| <= 2^-8 |v|, and
// v - v0 - v1 holds at most 8, which bf16 keeps (exponent range aside).  A
// product a b is then the six terms a_i b_j with i + j <= 2, each exact in
// the float32 accumulator's multiply; the three left out (a1 b2, a2 b1,
// a2 b2) total at most ~2^-23 |a b|, the size of float32's own rounding of a
// product.  Summed smallest first: (1,1), (0,2), (2,0), (0,1), (1,0), (0,0).
#pragma once
#include <hip/hip_runtime.h>

typedef __bf16 bx3_bf2 __attribute__((ext_vector_type(2)));
typedef __bf16 bx3_bf8 __attribute__((ext_vector_type(8)));
typedef float bx3_f2 __attribute__((ext_vector_type(2)));
typedef unsigned bx3_u4 __attribute__((ext_vector_type(4)));

// the (i, j) of the six kept terms, smallest first
__device__ constexpr int BX3_TA[6] = {1, 0, 2, 0, 1, 0};
__device__ constexpr int BX3_TB[6] = {1, 2, 0, 1, 0, 0};

// scale * v rounded to float32 before the split.  The empty asm makes the
// products opaque, so the compiler cannot contract them into the split's
// first subtraction (an FMA there would split the unrounded product, and two
// kernels could then disagree in the last bits).
__device__ __forceinline__ bx3_f2 bx3_scale2(bx3_f2 v, float s) {
  float a = v.x * s, b = v.y * s;
  asm volatile("" : "+v"(a), "+v"(b));
  return bx3_f2{a, b};
}

// two values -> their three terms as packed bf16 pairs (h[p] = term p of
// (v.x, v.y), low half v.x); float -> bf16 rounds to nearest even
// (v_cvt_pk_bf16_f32)
__device__ __forceinline__ void bx3_split2(bx3_f2 v, unsigned* h) {
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    const bx3_bf2 b = __builtin_convertvector(v, bx3_bf2);
    h[p] = __builtin_bit_cast(unsigned, b);
    if (p < 2) v -= bx3_f2{__uint_as_float(h[p] << 16), __uint_as_float(h[p] & 0xffff0000u)};
  }
}

// eight values (v[0..7]) -> three MFMA operands of 8 bf16, term p in t[p]
__device__ __forceinline__ void bx3_split8(const float* v, bx3_bf8* t) {
  bx3_u4 o[3];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    unsigned h[3];
    bx3_split2(bx3_f2{v[2 * e], v[2 * e + 1]}, h);
#pragma unroll
    for (int p = 0; p < 3; ++p) o[p][e] = h[p];
  }
#pragma unroll
  for (int p = 0; p < 3; ++p) t[p] = __builtin_bit_cast(bx3_bf8, o[p]);
}
