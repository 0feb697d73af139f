// Shared device helpers of the TECE kernels (tece_*.hip): per-edge
// wavefronts and head sums, the SO(2) block layout of the edge features, the
// l blocks of the edge-frame Wigner matrices, channel-pair loads and stores,
// and the block-pointer arguments of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"

int tace_fail_msg(const char* msg);   // tace_hip.hip
int tace_check_launch(const char* what);

// ------------------------------------------------------- per-edge wavefronts --
// The score, rotate-in and rotate-out backward kernels give each edge one
// wavefront (4 edges per 256-thread workgroup): lane l holds channels
// c = l + 64 j of slot j, so every feature row of an edge is one coalesced
// 256-byte (fp32) access and the edge's Wigner matrix is wave-uniform.
__device__ __forceinline__ int64_t wave_edge() {
  return (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Channel slots per lane for `C` channels (a compile-time bound of the loops).
#define TACE_SLOTS_DISPATCH(C, NS, ...)      \
  if ((C) <= 64) { constexpr int NS = 1; __VA_ARGS__; }       \
  else if ((C) <= 128) { constexpr int NS = 2; __VA_ARGS__; } \
  else if ((C) <= 256) { constexpr int NS = 4; __VA_ARGS__; } \
  else if ((C) <= 512) { constexpr int NS = 8; __VA_ARGS__; } \
  else { constexpr int NS = 16; __VA_ARGS__; }

// Sum over the lanes of one head of per-slot values v[0..V): heads of Ch < 64
// channels (Ch divides 64) are lane groups of one slot; heads of Ch >= 64
// (a multiple of 64) are whole slots, summed over the wave after their last
// slot.  `run` carries the partial sums of a wide head across slots.
// Returns true on the one lane (per head) that holds the total in v.
template <typename T, int V>
__device__ __forceinline__ bool head_sum(T* v, T* run, int j, int Ch, int lane) {
  if (Ch < 64) {
#pragma unroll
    for (int i = 0; i < V; ++i)
      for (int o = Ch >> 1; o > 0; o >>= 1) v[i] += __shfl_xor(v[i], o, 64);
    return (lane & (Ch - 1)) == 0;
  }
#pragma unroll
  for (int i = 0; i < V; ++i) run[i] += v[i];
  if (((j + 1) * 64) % Ch) return false;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    v[i] = wave_sum(run[i]);
    run[i] = T(0);
  }
  return lane == 0;
}

// ------------------------------------------------------ SO(2) block layout --
// Edge features of the convolution are kept as one 2-D GEMM operand per m
// (the "block layout"): block 0 is [E, (L+1) ch] (rows l = 0..L of m = 0) and
// block m > 0 is [2E, (L+1-m) ch], GEMM row 2e holding the +m rows of edge e
// and row 2e+1 its -m rows.  Row r of an edge's m layout (m = 0 rows, then per
// m the +m rows and the -m rows) is block mblk(r), local row mloc(r) of the
// edge's mrows(b) rows.  Kernels take the L+1 block pointers by value.
template <typename T>
struct Blk {
  T* p[4];
};

// Outputs that feed the SO(2)-linear GEMMs may be stored as bfloat16 (the
// bf16 channel-mixing option): round to nearest even, as torch's cast does,
// so the GEMM sees the operand it would get from a float32 output + cast.
typedef uint16_t bf16_t;
template <typename TO, typename T>
__device__ __forceinline__ TO out_cvt(T v) { return (TO)v; }
template <>
__device__ __forceinline__ bf16_t out_cvt<bf16_t, float>(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

template <int L>
__device__ __forceinline__ constexpr int mblk(int r) {
  if (r <= L) return 0;
  int off = L + 1;
  for (int m = 1; m <= L; ++m) {
    if (r < off + 2 * (L + 1 - m)) return m;
    off += 2 * (L + 1 - m);
  }
  return -1;
}

template <int L>
__device__ __forceinline__ constexpr int mstart(int b) {
  int off = 0;
  for (int m = 0; m < b; ++m) off += m == 0 ? L + 1 : 2 * (L + 1 - m);
  return off;
}

template <int L>
__device__ __forceinline__ constexpr int mrows(int b) { return b == 0 ? L + 1 : 2 * (L + 1 - b); }

// pointer to row r of edge e (channel 0) in a block array with `ch` channels
template <int L, typename T>
__device__ __forceinline__ T* erow(const Blk<T>& B, int64_t e, int r, int ch) {
  const int b = mblk<L>(r);
  return B.p[b] + (e * mrows<L>(b) + (r - mstart<L>(b))) * (int64_t)ch;
}

// the component (per m-layout row) of the radial weights w[e, comp, 2C]
template <int L>
__device__ __forceinline__ int m_comp(int r) {
  constexpr int n = L + 1;
  if (r < n) return r;
  int off = n, coff = n;
#pragma unroll
  for (int m = 1; m <= L; ++m) {
    const int k = n - m;
    if (r < off + 2 * k) return coff + (r - off < k ? r - off : r - off - k);
    off += 2 * k;
    coff += k;
  }
  return -1;
}

// The Wigner matrix is block-diagonal: row r of the m layout and column k of
// the l layout meet in a block when m_l(r) == l_of(k); the kernels read the
// blocks only.
template <int L>
__device__ __forceinline__ constexpr int m_l(int r) {   // l of m-layout row r
  if (r <= L) return r;
  int off = L + 1;
  for (int m = 1; m <= L; ++m) {
    const int n = L + 1 - m;
    if (r < off + 2 * n) return m + (r - off < n ? r - off : r - off - n);
    off += 2 * n;
  }
  return 0;
}

__device__ __forceinline__ constexpr int l_of(int k) {   // l of l-layout component k
  int l = 0;
  while ((l + 1) * (l + 1) <= k) ++l;
  return l;
}

// the i-th m-layout row of block l (i < 2l + 1, rows in increasing order:
// m = 0, then +1, -1, +2, -2, ...)
template <int L>
__device__ __forceinline__ constexpr int blk_row(int l, int i) {
  if (i == 0) return l;
  const int m = (i + 1) / 2;
  int off = L + 1;
  for (int mm = 1; mm < m; ++mm) off += 2 * (L + 1 - mm);
  return off + (i & 1 ? 0 : L + 1 - m) + (l - m);
}

template <int L>
__device__ __forceinline__ constexpr int wig_nb() {   // entries of the l blocks
  int s = 0;
  for (int l = 0; l <= L; ++l) s += (2 * l + 1) * (2 * l + 1);
  return s;
}

template <int L>
__device__ __forceinline__ constexpr int wig_row_off(int r) {   // first compact entry of row r
  int o = 0;
  for (int i = 0; i < r; ++i) o += 2 * m_l<L>(i) + 1;
  return o;
}

template <typename T, int V>
__device__ __forceinline__ void ldv(const T* p, T (&o)[V]) {
  if constexpr (V == 2) {
    static_assert(sizeof(T) == 4, "two channels per lane: float32 only");
    const float2 t = *(const float2*)p;
    o[0] = t.x;
    o[1] = t.y;
  } else {
    o[0] = *p;
  }
}

template <typename T, int V>
__device__ __forceinline__ void stv(T* p, const T (&o)[V]) {
  if constexpr (V == 2)
    *(float2*)p = make_float2(o[0], o[1]);
  else
    *p = o[0];
}

// one converted output element as a streamed (non-temporal) store
template <typename TO, typename T>
__device__ __forceinline__ void st_nt(TO* p, T v) {
  __builtin_nontemporal_store(out_cvt<TO>(v), p);
}

// the same into global memory as streamed (non-temporal) stores: per-edge
// outputs read once by a later kernel, so L2 stays with the gathered rows
typedef float tece_f2_t __attribute__((ext_vector_type(2)));
template <typename T, int V>
__device__ __forceinline__ void stv_nt(T* p, const T (&o)[V]) {
  if constexpr (V == 2)
    __builtin_nontemporal_store(tece_f2_t{o[0], o[1]}, (tece_f2_t*)p);
  else
    __builtin_nontemporal_store(o[0], p);
}

// ---------------------------------------------------------- C ABI helpers --
// block arrays: lmax+1 pointers (block 0, then m = 1..lmax); entries past
// lmax are ignored
template <typename T>
static Blk<T> blocks_of(const void* const* a, int lmax) {
  Blk<T> b{{nullptr, nullptr, nullptr, nullptr}};
  if (a)
    for (int m = 0; m <= lmax && m < 4; ++m) b.p[m] = (T*)a[m];
  return b;
}

static bool blocks_ok(const void* const* a, int lmax) {
  if (!a) return false;
  for (int m = 0; m <= lmax; ++m)
    if (!a[m]) return false;
  return true;
}

// one wavefront per edge, four per workgroup
static dim3 wave_grid(int64_t E) { return dim3((unsigned)((E + 3) / 4)); }

