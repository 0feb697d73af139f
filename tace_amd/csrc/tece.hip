// MI355X (gfx950) kernels of the TECE radial-rotary edge attention
// (tace/models/_e3nn/archive/oam_2026_07_05.py:547-823):
//   * edge-frame Wigner matrices in the SO(2) "m layout" from the edge vector
//     (tace/models/o2/rotation_matrix.py:74-88, tace/models/o2/wigner.py:231-357),
//     forward and the exact backward to the edge vector (reverse mode through
//     the D^l recursion, dual numbers for the frame);
//   * the radial-rotary complex QK score (oam_2026_07_05.py:699-754);
//   * the graph softmax over each receiver's in-edges (tace/models/softmax.py:100-112),
//     walked along the receiver CSR (no atomics);
//   * the attention-weighted inverse rotation and receiver sum of the
//     messages (oam_2026_07_05.py:799-823), CSR, written in the group-major
//     node layout.
// Exported through the C ABI of include/tace_hip.h.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"
#include "gen/wigner.inc"

int tace_fail_msg(const char* msg);   // tace_hip.hip
int tace_check_launch(const char* what);

// ------------------------------------------------------------ dual numbers --
// value and the three partial derivatives with respect to the edge vector
template <typename T>
struct Dual3 {
  T v, d[3];
  __device__ Dual3() : v(0), d{0, 0, 0} {}
  __device__ Dual3(T x) : v(x), d{0, 0, 0} {}
};
template <typename T>
__device__ __forceinline__ Dual3<T> operator+(const Dual3<T>& a, const Dual3<T>& b) {
  Dual3<T> r; r.v = a.v + b.v;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = a.d[i] + b.d[i];
  return r;
}
template <typename T>
__device__ __forceinline__ Dual3<T> operator-(const Dual3<T>& a, const Dual3<T>& b) {
  Dual3<T> r; r.v = a.v - b.v;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = a.d[i] - b.d[i];
  return r;
}
template <typename T>
__device__ __forceinline__ Dual3<T> operator-(const Dual3<T>& a) {
  Dual3<T> r; r.v = -a.v;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = -a.d[i];
  return r;
}
template <typename T>
__device__ __forceinline__ Dual3<T> operator*(const Dual3<T>& a, const Dual3<T>& b) {
  Dual3<T> r; r.v = a.v * b.v;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = a.d[i] * b.v + a.v * b.d[i];
  return r;
}
template <typename T>
__device__ __forceinline__ Dual3<T> operator/(const Dual3<T>& a, const Dual3<T>& b) {
  Dual3<T> r; const T ib = T(1) / b.v; r.v = a.v * ib;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = (a.d[i] - r.v * b.d[i]) * ib;
  return r;
}
template <typename T> __device__ __forceinline__ T val(T x) { return x; }
template <typename T> __device__ __forceinline__ T val(const Dual3<T>& x) { return x.v; }
template <typename T> __device__ __forceinline__ T f_sqrt(T x) { return sqrt(x); }
template <typename T> __device__ __forceinline__ Dual3<T> f_sqrt(const Dual3<T>& a) {
  Dual3<T> r; r.v = sqrt(a.v); const T h = T(0.5) / r.v;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = a.d[i] * h;
  return r;
}
template <typename T> __device__ __forceinline__ T f_exp(T x) { return exp(x); }
template <typename T> __device__ __forceinline__ Dual3<T> f_exp(const Dual3<T>& a) {
  Dual3<T> r; r.v = exp(a.v);
#pragma unroll
  for (int i = 0; i < 3; ++i) r.d[i] = a.d[i] * r.v;
  return r;
}

// ------------------------------------------------------------- edge frame --
// Rotation R (row-major) taking the edge direction to +y: unit quaternions of
// two charts, q+ = (1+y, -z, 0, x) and q- = (-z, 1-y, x, 0) in (w, x, y, z),
// blended by nlerp with the C-infinity step s((y+1)/2); norms carry eps = 1e-7
// inside the square root (rotation_matrix.py:16-88).
template <typename T, typename S>
__device__ __forceinline__ S nrm4(const S& a, const S& b, const S& c, const S& d) {
  return f_sqrt(a * a + b * b + c * c + d * d + S(T(1e-14)));
}

template <typename T, typename S>
__device__ void edge_frame(const S& vx, const S& vy, const S& vz, S* R) {
  const S n = f_sqrt(vx * vx + vy * vy + vz * vz + S(T(1e-14)));
  const S x = vx / n, y = vy / n, z = vz / n;
  const S one(T(1)), zero(T(0));
  S p0 = one + y, p1 = -z, p2 = zero, p3 = x;
  S np = nrm4<T>(p0, p1, p2, p3);
  p0 = p0 / np; p1 = p1 / np; p3 = p3 / np;
  S q0 = -z, q1 = one - y, q2 = x, q3 = zero;
  S nq = nrm4<T>(q0, q1, q2, q3);
  q0 = q0 / nq; q1 = q1 / nq; q2 = q2 / nq;
  // smooth step t(s), s = (y + 1) / 2 clamped to [0, 1]
  S s = S(T(0.5)) * (y + one);
  S t;
  const T tiny = sizeof(T) == 4 ? T(1.1920928955078125e-07) : T(2.220446049250313e-16);
  if (val(s) <= T(0)) {
    t = zero;
  } else if (val(s) >= T(1)) {
    t = one;
  } else {
    const S sa = val(s) < tiny ? S(tiny) : s;
    const S sb = val(one - s) < tiny ? S(tiny) : one - s;
    const S a = f_exp(-(one / sa)), b = f_exp(-(one / sb));
    t = a / (a + b);
  }
  if (val(q0 * p0 + q1 * p1 + q2 * p2 + q3 * p3) < T(0)) {
    p0 = -p0; p1 = -p1; p2 = -p2; p3 = -p3;
  }
  const S u = one - t;
  S w = u * q0 + t * p0, a = u * q1 + t * p1, b = u * q2 + t * p2, c = u * q3 + t * p3;
  const S nn = nrm4<T>(w, a, b, c);
  w = w / nn; a = a / nn; b = b / nn; c = c / nn;
  const S two(T(2));
  R[0] = one - two * (b * b + c * c); R[1] = two * (a * b - w * c); R[2] = two * (a * c + w * b);
  R[3] = two * (a * b + w * c); R[4] = one - two * (a * a + c * c); R[5] = two * (b * c - w * a);
  R[6] = two * (a * c - w * b); R[7] = two * (b * c + w * a); R[8] = one - two * (a * a + b * b);
}

// D^L [dn x dn] = (2L+1) sum cg[a][b][m] R[a][c] P[b][d] cg[c][d][n], with
// P = D^(L-1) and cg = W3j(1, L-1, L) (wigner.py:330-357).
template <typename T, typename S, int L>
__device__ void wig_next(const S* R, const S* P, S* D) {
  constexpr int dp = 2 * L - 1, dn = 2 * L + 1;
  const double* cg = WigCG<L>::v;
  S U[dn][3][dp];
#pragma unroll
  for (int m = 0; m < dn; ++m)
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
      for (int d = 0; d < dp; ++d) U[m][c][d] = S(T(0));
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < dp; ++b)
#pragma unroll
      for (int m = 0; m < dn; ++m) {
        const double k = cg[(a * dp + b) * dn + m];
        if (k != 0.0) {
#pragma unroll
          for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int d = 0; d < dp; ++d) U[m][c][d] = U[m][c][d] + S(T(k)) * R[a * 3 + c] * P[b * dp + d];
        }
      }
#pragma unroll
  for (int m = 0; m < dn; ++m)
#pragma unroll
    for (int n = 0; n < dn; ++n) {
      S acc(T(0));
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int d = 0; d < dp; ++d) {
          const double k = cg[(c * dp + d) * dn + n];
          if (k != 0.0) acc = acc + S(T(k)) * U[m][c][d];
        }
      D[m * dn + n] = S(T(2 * L + 1)) * acc;
    }
}

// e3nn component index (l^2 + l + m) of row r of the m layout (mmax = L):
// m = 0 for l = 0..L, then per m the +m rows and the -m rows (wigner.py:38-66)
template <int L>
__device__ __forceinline__ int m_row(int r) {
  int off = L + 1;
  if (r < off) return r * r + r;
  for (int m = 1; m <= L; ++m) {
    const int n = L + 1 - m;
    if (r < off + n) { const int l = m + (r - off); return l * l + l + m; }
    if (r < off + 2 * n) { const int l = m + (r - off - n); return l * l + l - m; }
    off += 2 * n;
  }
  return -1;
}

// W [K x K], K = (L+1)^2: row r = block-diagonal Wigner row m_row(r)
template <typename T, typename S, int L>
__device__ void wigner_m(const S& vx, const S& vy, const S& vz, S* W) {
  constexpr int K = (L + 1) * (L + 1);
  S R[9];
  edge_frame<T>(vx, vy, vz, R);
  S D2[25], D3[49];
  if (L >= 2) wig_next<T, S, 2>(R, R, D2);
  if (L >= 3) wig_next<T, S, 3>(R, D2, D3);
#pragma unroll
  for (int r = 0; r < K; ++r) {
    const int src = m_row<L>(r);
    int l = 0;
    while ((l + 1) * (l + 1) <= src) ++l;
    const int i = src - l * l;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      int lk = 0;
      while ((lk + 1) * (lk + 1) <= k) ++lk;
      const int j = k - lk * lk;
      S v(T(0));
      if (lk == l) {
        if (l == 0) v = S(T(1));
        else if (l == 1) v = R[i * 3 + j];
        else if (l == 2) v = D2[i * 5 + j];
        else v = D3[i * 7 + j];
      }
      W[r * K + k] = v;
    }
  }
}

// Adjoint of wig_next: given gD = dE/dD, accumulate dE/dR into gR and dE/dP
// into gP (U is linear in R and in P, D linear in U); one row m of U at a time.
template <typename T, int L>
__device__ void wig_next_adj(const T* R, const T* P, const T* gD, T* gR, T* gP) {
  constexpr int dp = 2 * L - 1, dn = 2 * L + 1;
  const double* cg = WigCG<L>::v;
#pragma unroll
  for (int m = 0; m < dn; ++m) {
    T gU[3][dp];
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
      for (int d = 0; d < dp; ++d) {
        T acc = T(0);
#pragma unroll
        for (int n = 0; n < dn; ++n) {
          const double k = cg[(c * dp + d) * dn + n];
          if (k != 0.0) acc += T(k) * gD[m * dn + n];
        }
        gU[c][d] = T(2 * L + 1) * acc;
      }
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < dp; ++b) {
        const double k = cg[(a * dp + b) * dn + m];
        if (k != 0.0) {
#pragma unroll
          for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int d = 0; d < dp; ++d) {
              gR[a * 3 + c] += T(k) * gU[c][d] * P[b * dp + d];
              gP[b * dp + d] += T(k) * R[a * 3 + c] * gU[c][d];
            }
        }
      }
  }
}

// Forward: one edge per lane; a wavefront's 64 matrices go through LDS (row
// stride K*K+1 words, odd or padded, so the per-lane writes hit distinct banks)
// and leave as one contiguous, coalesced run. Matrices too large for 64 KB of
// LDS are stored per lane.
template <typename T, int L>
__global__ __launch_bounds__(64) void k_wigner_fwd(const T* __restrict__ vec, int64_t E, T* __restrict__ W) {
  constexpr int K = (L + 1) * (L + 1), KK = K * K;
  constexpr int KP = (KK % 2) ? KK : KK + 1;
  constexpr bool STAGE = 64 * KP * sizeof(T) <= 65536;
  const int64_t e0 = (int64_t)blockIdx.x * 64;
  const int64_t e = e0 + threadIdx.x;
  T w[KK];
  if (e < E) wigner_m<T, T, L>(vec[3 * e], vec[3 * e + 1], vec[3 * e + 2], w);
  if constexpr (STAGE) {
    __shared__ T st[64 * KP];
#pragma unroll
    for (int i = 0; i < KK; ++i) st[threadIdx.x * KP + i] = w[i];
    __syncthreads();
    const int nv = E - e0 < 64 ? (int)(E - e0) : 64;
    T* o = W + e0 * KK;
    for (int idx = threadIdx.x; idx < nv * KK; idx += 64) o[idx] = st[(idx / KK) * KP + idx % KK];
  } else {
    if (e >= E) return;
    T* o = W + e * KK;
#pragma unroll
    for (int i = 0; i < KK; ++i) o[i] = w[i];
  }
}

// Backward, reverse mode: the incoming gradient is read on the diagonal blocks
// only (the others multiply constant zeros), pulled back through the D^l
// recursion to the frame R, and R's dual parts (forward mode over the three
// vector components) take it to the edge vector.
template <typename T, int L>
__global__ __launch_bounds__(64) void k_wigner_bwd(const T* __restrict__ vec, const T* __restrict__ gW, int64_t E,
                                                   T* __restrict__ gv) {
  constexpr int K = (L + 1) * (L + 1);
  const int64_t e = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (e >= E) return;
  Dual3<T> x(vec[3 * e]), y(vec[3 * e + 1]), z(vec[3 * e + 2]);
  x.d[0] = T(1); y.d[1] = T(1); z.d[2] = T(1);
  Dual3<T> Rd[9];
  edge_frame<T>(x, y, z, Rd);
  T R[9], gR[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) { R[k] = Rd[k].v; gR[k] = T(0); }
  T gD2[25], gD3[49];
  const T* g = gW + e * K * K;
#pragma unroll
  for (int r = 0; r < K; ++r) {
    const int src = m_row<L>(r);
    int l = 0;
    while ((l + 1) * (l + 1) <= src) ++l;
    const int i = src - l * l;
#pragma unroll
    for (int j = 0; j < 2 * l + 1; ++j) {
      const T v = g[r * K + l * l + j];
      if (l == 1) gR[i * 3 + j] += v;
      else if (l == 2) gD2[i * 5 + j] = v;
      else if (l == 3) gD3[i * 7 + j] = v;
    }
  }
  if constexpr (L >= 3) {
    T D2[25];
    wig_next<T, T, 2>(R, R, D2);
    wig_next_adj<T, 3>(R, D2, gD3, gR, gD2);
  }
  if constexpr (L >= 2) {
    T gP[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) gP[k] = T(0);
    wig_next_adj<T, 2>(R, R, gD2, gR, gP);
#pragma unroll
    for (int k = 0; k < 9; ++k) gR[k] += gP[k];
  }
  T a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    a0 += gR[k] * Rd[k].d[0]; a1 += gR[k] * Rd[k].d[1]; a2 += gR[k] * Rd[k].d[2];
  }
  gv[3 * e] = a0; gv[3 * e + 1] = a1; gv[3 * e + 2] = a2;
}

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

// -------------------------------------------------------------- QK score --
// score[e,h] = (S0 + sum_m cos(m phi) A_m + sin(m phi) B_m) * tscale[h] + rp[e,h],
// phi = pi tanh(rp[e, H+h]);  S0 = sum over the m = 0 rows of q.k,
// A_m = sum(q_re k_re + q_im k_im), B_m = sum(q_im k_re - q_re k_im) over the
// +-m rows (rows re..re+n-1 and re+n..re+2n-1, n = L+1-m) and the head's Ch
// channels.  Rows of the m layout: m = 0 rows 0..L, then per m the +m and -m rows.
template <int L>
__device__ __forceinline__ int m_rows_start(int m) {
  int off = L + 1;
  for (int mm = 1; mm < m; ++mm) off += 2 * (L + 1 - mm);
  return off;
}

template <typename T, int L, int NS>
__global__ __launch_bounds__(256) void k_score_fwd(const Blk<const T> q, const Blk<const T> k,
                                                   const T* __restrict__ rp, const T* __restrict__ tscale,
                                                   int64_t E, int C, int H, T* __restrict__ score) {
  constexpr int V = 1 + 2 * L;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const int Ch = C / H;
  T run[V];
#pragma unroll
  for (int i = 0; i < V; ++i) run[i] = T(0);
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j >= C) break;
    const int c = lane + 64 * j;
    T v[V];
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = T(0);
    if (c < C) {
#pragma unroll
      for (int r = 0; r <= L; ++r) v[0] += erow<L>(q, e, r, C)[c] * erow<L>(k, e, r, C)[c];
#pragma unroll
      for (int m = 1; m <= L; ++m) {
        const int re = m_rows_start<L>(m), n = L + 1 - m;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          const T qr = erow<L>(q, e, re + i, C)[c], qi = erow<L>(q, e, re + n + i, C)[c];
          const T kr = erow<L>(k, e, re + i, C)[c], ki = erow<L>(k, e, re + n + i, C)[c];
          v[2 * m - 1] += qr * kr + qi * ki;
          v[2 * m] += qi * kr - qr * ki;
        }
      }
    }
    if (head_sum<T, V>(v, run, j, Ch, lane) && c < C) {
      const int h = c / Ch;
      const T phi = T(M_PI) * tanh(rp[e * 2 * H + H + h]);
      T s = v[0];
#pragma unroll
      for (int m = 1; m <= L; ++m) s += cos(T(m) * phi) * v[2 * m - 1] + sin(T(m) * phi) * v[2 * m];
      score[e * H + h] = s * tscale[h] + rp[e * 2 * H + h];
    }
  }
}

template <typename T, typename TO, int L, int NS>
__global__ __launch_bounds__(256) void k_score_bwd(const Blk<const T> q, const Blk<const T> k,
                                                   const T* __restrict__ rp, const T* __restrict__ tscale,
                                                   const T* __restrict__ gs, int64_t E, int C, int H,
                                                   const Blk<TO> gq, const Blk<TO> gk, T* __restrict__ grp) {
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const int Ch = C / H;
  T run[1] = {T(0)};
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j >= C) break;
    const int c = lane + 64 * j;
    const bool act = c < C;
    const int h = act ? c / Ch : 0;
    const T g = gs[e * H + h];
    const T G = g * tscale[h];
    const T th = tanh(rp[e * 2 * H + H + h]);
    const T phi = T(M_PI) * th;
    T d[1] = {T(0)};
    if (act) {
#pragma unroll
      for (int r = 0; r <= L; ++r) {
        const T qv = erow<L>(q, e, r, C)[c], kv = erow<L>(k, e, r, C)[c];
        erow<L>(gq, e, r, C)[c] = out_cvt<TO>(G * kv);
        erow<L>(gk, e, r, C)[c] = out_cvt<TO>(G * qv);
      }
#pragma unroll
      for (int m = 1; m <= L; ++m) {
        const int re = m_rows_start<L>(m), n = L + 1 - m;
        const T cs = cos(T(m) * phi), sn = sin(T(m) * phi);
        T A = 0, B = 0;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          const int ir = re + i, ii = re + n + i;
          const T qr = erow<L>(q, e, ir, C)[c], qi = erow<L>(q, e, ii, C)[c];
          const T kr = erow<L>(k, e, ir, C)[c], ki = erow<L>(k, e, ii, C)[c];
          A += qr * kr + qi * ki;
          B += qi * kr - qr * ki;
          erow<L>(gq, e, ir, C)[c] = out_cvt<TO>(G * (cs * kr - sn * ki));
          erow<L>(gq, e, ii, C)[c] = out_cvt<TO>(G * (cs * ki + sn * kr));
          erow<L>(gk, e, ir, C)[c] = out_cvt<TO>(G * (cs * qr + sn * qi));
          erow<L>(gk, e, ii, C)[c] = out_cvt<TO>(G * (cs * qi - sn * qr));
        }
        d[0] += T(m) * (cs * B - sn * A);
      }
    }
    if (head_sum<T, 1>(d, run, j, Ch, lane) && act) {
      grp[e * 2 * H + h] = g;
      grp[e * 2 * H + H + h] = G * d[0] * T(M_PI) * (T(1) - th * th);
    }
  }
}

// ----------------------------------------------------- rotate into the frame --
// m[e, r, c] = sum_k W[e, r, k] x[row(e, c), k, c mod C] over the 2C channels
// of [x_src | x_dst]: row = rows_src[e] for c < C, rows_dst[e] otherwise
// (the gather, concatenation and wigner bmm of oam_2026_07_05.py:769-771).
// Outputs: ms = m[:, :, :C] and md = m[:, :, C:] (contiguous [E, K, C] each,
// the key / query projection inputs) and, when radial weights w [E, ncomp, 2C]
// are given, mw = w[e, comp(r), c] m[e, r, c] ([E, K, 2C], the radial
// weighting of oam_2026_07_05.py:778-780: +m and -m rows share a component).
// x: [n_rows, K, C] node features in the l layout; rows outside [0, n_rows)
// read as zeros.
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

template <typename T, typename TO, int L, int NS>
__global__ __launch_bounds__(256) void k_rotin_fwd(const T* __restrict__ x, const T* __restrict__ W,
                                                   const int64_t* __restrict__ rows_src,
                                                   const int64_t* __restrict__ rows_dst, const T* __restrict__ wr,
                                                   int64_t n_rows, int64_t E, int C, const Blk<TO> ms,
                                                   const Blk<TO> md, const Blk<TO> mw) {
  constexpr int K = (L + 1) * (L + 1), NC = (L + 1) * (L + 2) / 2;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const T* w = W + e * K * K;
  const int64_t rs = rows_src[e], rd = rows_dst[e];
  const int C2 = 2 * C;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j >= C2) break;
    const int c = lane + 64 * j;
    if (c >= C2) continue;
    const bool src = c < C;
    const int64_t row = src ? rs : rd;
    const int cc = src ? c : c - C;
    T xk[K];
    const bool ok = row >= 0 && row < n_rows;
#pragma unroll
    for (int kk = 0; kk < K; ++kk) xk[kk] = ok ? x[(row * K + kk) * C + cc] : T(0);
#pragma unroll
    for (int r = 0; r < K; ++r) {
      T a = 0;
#pragma unroll
      for (int kk = 0; kk < K; ++kk) a += w[r * K + kk] * xk[kk];
      erow<L>(src ? ms : md, e, r, C)[cc] = out_cvt<TO>(a);
      if (wr) erow<L>(mw, e, r, C2)[c] = out_cvt<TO>(wr[(e * NC + m_comp<L>(r)) * C2 + c] * a);
    }
  }
}

// The same forward for float32 features and an even channel count, two
// adjacent channels per lane: 8-byte feature and radial-weight loads and
// 4-byte (bf16) or 8-byte (float32) stores, half the memory instructions of
// the kernel above.  Each output row sums over its own l block of the
// block-diagonal Wigner matrix only: the other entries are zeros, whose
// products the kernel above adds (fma(0, x, a) = a), so the sums are the same
// bits.  Needs x and radial_w 8-byte aligned and the output blocks aligned to
// two elements.
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

__device__ __forceinline__ void st_pair(float* p, float a, float b) { *(float2*)p = make_float2(a, b); }
__device__ __forceinline__ void st_pair(bf16_t* p, float a, float b) {
  *(uint32_t*)p = (uint32_t)out_cvt<bf16_t>(a) | ((uint32_t)out_cvt<bf16_t>(b) << 16);
}

template <typename TO, int L, int NP>
__global__ __launch_bounds__(256) void k_rotin_fwd_pairs(const float* __restrict__ x, const float* __restrict__ W,
                                                         const int64_t* __restrict__ rows_src,
                                                         const int64_t* __restrict__ rows_dst,
                                                         const float* __restrict__ wr, int64_t n_rows, int64_t E,
                                                         int C, const Blk<TO> ms, const Blk<TO> md,
                                                         const Blk<TO> mw) {
  constexpr int K = (L + 1) * (L + 1), NC = (L + 1) * (L + 2) / 2;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const float* w = W + e * K * K;
  const int64_t rs = rows_src[e], rd = rows_dst[e];
  const int C2 = 2 * C;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int c = 2 * (lane + 64 * j);
    if (c < C2) {
      const bool src = c < C;
      const int64_t row = src ? rs : rd;
      const int cc = src ? c : c - C;
      const bool ok = row >= 0 && row < n_rows;
      float2 xk[K];
#pragma unroll
      for (int kk = 0; kk < K; ++kk)
        xk[kk] = ok ? *(const float2*)(x + (row * K + kk) * C + cc) : make_float2(0.f, 0.f);
#pragma unroll
      for (int r = 0; r < K; ++r) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int kk = 0; kk < K; ++kk) {
          if (l_of(kk) != m_l<L>(r)) continue;   // constant after unrolling
          a0 += w[r * K + kk] * xk[kk].x;
          a1 += w[r * K + kk] * xk[kk].y;
        }
        st_pair(erow<L>(src ? ms : md, e, r, C) + cc, a0, a1);
        if (wr) {
          const float2 wv = *(const float2*)(wr + (e * NC + m_comp<L>(r)) * C2 + c);
          st_pair(erow<L>(mw, e, r, C2) + c, wv.x * a0, wv.y * a1);
        }
      }
    }
  }
}

// Sums p[0..P) over the 64 lanes in groups of 16 (reduce16_lanes) and stores
// the totals at out[0..n).
template <typename T, int P>
__device__ __forceinline__ void store_lane_sums(const T* p, int n, T* out, int lane) {
#pragma unroll
  for (int g = 0; g < P / 16; ++g) {
    const T t = reduce16_lanes(p[16 * g], p[16 * g + 1], p[16 * g + 2], p[16 * g + 3], p[16 * g + 4],
                               p[16 * g + 5], p[16 * g + 6], p[16 * g + 7], p[16 * g + 8], p[16 * g + 9],
                               p[16 * g + 10], p[16 * g + 11], p[16 * g + 12], p[16 * g + 13], p[16 * g + 14],
                               p[16 * g + 15]);
    const int i = 16 * g + rev4(lane);
    if (lane < 16 && i < n) out[i] = t;
  }
}

// backward: with g[e,r,c] = g_ms / g_md [e,r,c mod C] + w[e,comp(r),c] g_mw[e,r,c]
// (absent gradients count as zero):
//   g_x_src[e, k, c] = sum_r W[e,r,k] g[e,r,c] (c < C), g_x_dst the same for
//   channels C..2C-1 (per edge; the caller sums them into the rows);
//   g_W[e, r, k] = sum over the 2C channels of g[e,r,c] x[row(e,c), k, c];
//   g_w[e, comp, c] = sum of g_mw[e,r,c] m[e,r,c] over the rows r of comp.
template <typename T, int L, int NS, bool RUNS>
__device__ __forceinline__ void rotin_bwd_edge(const T* __restrict__ x, const T* __restrict__ W,
                                               const int64_t* __restrict__ rows_src,
                                               const int64_t* __restrict__ rows_dst, const T* __restrict__ wr,
                                               const Blk<const T>& gms, const Blk<const T>& gmd,
                                               const Blk<const T>& gmw, int64_t n_rows, int64_t E, int C, int64_t e,
                                               T* __restrict__ gxs, T* __restrict__ gxd, T* __restrict__ gW,
                                               T* __restrict__ gwr, T* __restrict__ lrow) {
  constexpr int K = (L + 1) * (L + 1), P = (K * K + 15) / 16 * 16, NC = (L + 1) * (L + 2) / 2;
  const int lane = (int)threadIdx.x & 63;
  const T* w = W + e * K * K;
  const int64_t rs = rows_src[e], rd = rows_dst[e];
  const int C2 = 2 * C;
  T p[P];
#pragma unroll
  for (int i = 0; i < P; ++i) p[i] = T(0);
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j >= C2) break;
    const int c = lane + 64 * j;
    if (c < C2) {
      const bool src = c < C;
      const int64_t row = src ? rs : rd;
      const int cc = src ? c : c - C;
      const bool ok = row >= 0 && row < n_rows;
      const Blk<const T>& gsd = src ? gms : gmd;
      T xk[K], g[K];
#pragma unroll
      for (int kk = 0; kk < K; ++kk) xk[kk] = ok ? x[(row * K + kk) * C + cc] : T(0);
#pragma unroll
      for (int r = 0; r < K; ++r) g[r] = gsd.p[mblk<L>(r)] ? erow<L>(gsd, e, r, C)[cc] : T(0);
      if (wr) {
        T gc[NC];
#pragma unroll
        for (int q = 0; q < NC; ++q) gc[q] = T(0);
#pragma unroll
        for (int r = 0; r < K; ++r) {
          const T gr = gmw.p[mblk<L>(r)] ? erow<L>(gmw, e, r, C2)[c] : T(0);
          const int q = m_comp<L>(r);
          g[r] += wr[(e * NC + q) * C2 + c] * gr;
          T mv = 0;
#pragma unroll
          for (int kk = 0; kk < K; ++kk) mv += w[r * K + kk] * xk[kk];
          gc[q] += gr * mv;
        }
        if (gwr) {
#pragma unroll
          for (int q = 0; q < NC; ++q) gwr[(e * NC + q) * C2 + c] = gc[q];
        }
      }
#pragma unroll
      for (int kk = 0; kk < K; ++kk) {
        T a = 0;
#pragma unroll
        for (int r = 0; r < K; ++r) a += w[r * K + kk] * g[r];
        if (RUNS && !src)
          lrow[kk * C + cc] = a;
        else
          (src ? gxs : gxd)[(e * K + kk) * C + cc] = a;
      }
#pragma unroll
      for (int r = 0; r < K; ++r)
#pragma unroll
        for (int kk = 0; kk < K; ++kk) p[r * K + kk] += g[r] * xk[kk];
    }
  }
  store_lane_sums<T, P>(p, K * K, gW + e * K * K, lane);
}

// One edge per wavefront (4 per workgroup).
// RUNS (edges in receiver-CSR order, dynamic LDS of 4 K C values): the four
// edges of a workgroup put their receiver rows in LDS, and each run of edges
// with the same receiver row writes one row, the run's sum in edge order, at
// the run's first position; positions inside a run are left unwritten.  A
// run starts at a receiver's first edge or at a multiple of 4, which is what
// tace_rows_accumulate_runs reads (run = 4).
template <typename T, int L, int NS, bool RUNS>
__global__ __launch_bounds__(256) void k_rotin_bwd(const T* __restrict__ x, const T* __restrict__ W,
                                                   const int64_t* __restrict__ rows_src,
                                                   const int64_t* __restrict__ rows_dst, const T* __restrict__ wr,
                                                   const Blk<const T> gms, const Blk<const T> gmd,
                                                   const Blk<const T> gmw, int64_t n_rows, int64_t E, int C,
                                                   T* __restrict__ gxs, T* __restrict__ gxd, T* __restrict__ gW,
                                                   T* __restrict__ gwr) {
  constexpr int K = (L + 1) * (L + 1);
  extern __shared__ __attribute__((aligned(16))) unsigned char rb_raw[];
  const int64_t e = wave_edge();
  if (!RUNS && e >= E) return;
  if (e < E) rotin_bwd_edge<T, L, NS, RUNS>(x, W, rows_src, rows_dst, wr, gms, gmd, gmw, n_rows, E, C, e, gxs, gxd, gW,
                                            gwr, (T*)rb_raw + (threadIdx.x >> 6) * K * C);
  if constexpr (RUNS) {
    __syncthreads();
    const T* rows = (const T*)rb_raw;
    const int64_t e0 = (int64_t)blockIdx.x * 4;
    const int KC = K * C;
    int64_t rd[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) rd[w] = e0 + w < E ? rows_dst[e0 + w] : -2;
    for (int w = 0; w < 4 && e0 + w < E; ++w) {
      if (w > 0 && rd[w] == rd[w - 1]) continue;   // inside a run
      int w1 = w + 1;
      while (w1 < 4 && rd[w1] == rd[w]) ++w1;
      for (int i = (int)threadIdx.x; i < KC; i += 256) {
        T v = rows[w * KC + i];
        for (int u = w + 1; u < w1; ++u) v += rows[u * KC + i];
        gxd[(e0 + w) * KC + i] = v;
      }
    }
  }
}

// ------------------------------------------------------------- edge ACE --
// Gate + complex edge-ACE product of the SO(2) messages
// (oam_2026_07_05.py:782-790, SO2Gate gate_m0 and uuuSO2TensorProduct
// 312-516, mmax = lmax = L, n = L+1 rows per m and sign, A hidden channels):
//   out = u + g u + ece(u, v, c)
// u = linear_up features, v = linear_glu features, g = ScaledSigmoid of the
// linear_up gate rows (row (m, i) of either sign takes gate m n + i), c =
// ScaledSigmoid of the linear_coefs output (one weight per path, row and
// channel).  ece: for every m3 the paths (m1 >= m2) with m1 + m2 = m3 ("sum",
// z = a b) or |m1 - m2| = m3 ("diff", z = a conj(b)), a from u at m1, b from
// v at m2 (m = 0 features are real), out re/im += z c, scaled by
// 1/sqrt(#paths of m3); m3 = 0 keeps the real part.
// Inputs are the stacked GEMM outputs: y0 [E, ncoef | n A (v, m=0) |
// (n (L+1) + n) A (gates, then u, m=0)] with ncoef = #paths n A, and for
// m > 0 y_m [2E, n A (v) | n A (u)] (row 2e = +m, 2e+1 = -m).  Outputs o0
// [E, n A] and o_m [2E, n A].  One thread per (edge, channel).
#define TACE_ACE_SCST 1.8467055342154763

template <int L>
struct AcePaths {
  static constexpr int count(int m3) {
    int c = 0;
    for (int m1 = 0; m1 <= L; ++m1)
      for (int m2 = 0; m2 <= m1; ++m2)
        if (m1 + m2 == m3 || m1 - m2 == m3) ++c;
    return c;
  }
  static constexpr int total() {
    int c = 0;
    for (int m3 = 0; m3 <= L; ++m3) c += count(m3);
    return c;
  }
};

template <typename T>
__device__ __forceinline__ T scaled_sigmoid(T z) { return T(TACE_ACE_SCST) / (T(1) + exp(-z)); }

template <typename T, typename TO, int L>
__global__ __launch_bounds__(256) void k_edge_ace_fwd(const T* __restrict__ y0, const T* __restrict__ y1,
                                                      const T* __restrict__ y2, const T* __restrict__ y3, int64_t E,
                                                      int A, TO* __restrict__ o0, TO* __restrict__ o1,
                                                      TO* __restrict__ o2, TO* __restrict__ o3) {
  constexpr int n = L + 1, NG = n * (L + 1), NP = AcePaths<L>::total();
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= E * A) return;
  const int64_t e = t / A;
  const int a = (int)(t - e * A);
  const T* ym[4] = {y0, y1, y2, y3};
  TO* om[4] = {o0, o1, o2, o3};
  const int64_t r0 = e * (int64_t)(NP * n * A + n * A + (NG + n) * A);
  const int cv0 = NP * n * A, cg = cv0 + n * A, cu0 = cg + NG * A;
  // u, v [m][sign][i]
  T u[L + 1][2][n], v[L + 1][2][n];
#pragma unroll
  for (int i = 0; i < n; ++i) {
    u[0][0][i] = y0[r0 + cu0 + i * A + a];
    v[0][0][i] = y0[r0 + cv0 + i * A + a];
    u[0][1][i] = T(0);
    v[0][1][i] = T(0);
  }
#pragma unroll
  for (int m = 1; m <= L; ++m)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < n; ++i) {
        const int64_t r = (2 * e + s) * (int64_t)(2 * n * A);
        v[m][s][i] = ym[m][r + i * A + a];
        u[m][s][i] = ym[m][r + n * A + i * A + a];
      }
  T re[L + 1][n], im[L + 1][n];
#pragma unroll
  for (int m = 0; m <= L; ++m)
#pragma unroll
    for (int i = 0; i < n; ++i) re[m][i] = im[m][i] = T(0);
  int p = 0;
#pragma unroll
  for (int m3 = 0; m3 <= L; ++m3)
#pragma unroll
    for (int m1 = 0; m1 <= L; ++m1)
#pragma unroll
      for (int m2 = 0; m2 <= m1; ++m2) {
        const bool sum = m1 + m2 == m3;
        if (!sum && m1 - m2 != m3) continue;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          const T w = scaled_sigmoid(y0[r0 + (p * n + i) * A + a]);
          const T ar = u[m1][0][i], ai = u[m1][1][i], br = v[m2][0][i], bi = v[m2][1][i];
          T zr, zi;
          if (sum) { zr = ar * br - ai * bi; zi = ar * bi + ai * br; }
          else { zr = ar * br + ai * bi; zi = ai * br - ar * bi; }
          re[m3][i] += zr * w;
          im[m3][i] += zi * w;
        }
        ++p;
      }
#pragma unroll
  for (int m3 = 0; m3 <= L; ++m3) {
    const T sc = T(1) / sqrt(T(AcePaths<L>::count(m3)));
#pragma unroll
    for (int i = 0; i < n; ++i) {
      const T g = scaled_sigmoid(y0[r0 + cg + (m3 * n + i) * A + a]);
      if (m3 == 0) {
        o0[e * (n * A) + i * A + a] = out_cvt<TO>(u[0][0][i] * (T(1) + g) + re[0][i] * sc);
      } else {
        om[m3][(2 * e) * (n * A) + i * A + a] = out_cvt<TO>(u[m3][0][i] * (T(1) + g) + re[m3][i] * sc);
        om[m3][(2 * e + 1) * (n * A) + i * A + a] = out_cvt<TO>(u[m3][1][i] * (T(1) + g) + im[m3][i] * sc);
      }
    }
  }
}

template <typename T, typename TO, int L>
__global__ __launch_bounds__(256) void k_edge_ace_bwd(const T* __restrict__ y0, const T* __restrict__ y1,
                                                      const T* __restrict__ y2, const T* __restrict__ y3,
                                                      const T* __restrict__ go0, const T* __restrict__ go1,
                                                      const T* __restrict__ go2, const T* __restrict__ go3, int64_t E,
                                                      int A, TO* __restrict__ gy0, TO* __restrict__ gy1,
                                                      TO* __restrict__ gy2, TO* __restrict__ gy3) {
  constexpr int n = L + 1, NG = n * (L + 1), NP = AcePaths<L>::total();
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= E * A) return;
  const int64_t e = t / A;
  const int a = (int)(t - e * A);
  const T* ym[4] = {y0, y1, y2, y3};
  const T* gom[4] = {go0, go1, go2, go3};
  TO* gym[4] = {gy0, gy1, gy2, gy3};
  const int64_t r0 = e * (int64_t)(NP * n * A + n * A + (NG + n) * A);
  const int cv0 = NP * n * A, cg = cv0 + n * A, cu0 = cg + NG * A;
  T u[L + 1][2][n], v[L + 1][2][n], go[L + 1][2][n], gu[L + 1][2][n], gv[L + 1][2][n];
#pragma unroll
  for (int i = 0; i < n; ++i) {
    u[0][0][i] = y0[r0 + cu0 + i * A + a];
    v[0][0][i] = y0[r0 + cv0 + i * A + a];
    go[0][0][i] = go0[e * (n * A) + i * A + a];
    u[0][1][i] = v[0][1][i] = go[0][1][i] = T(0);
  }
#pragma unroll
  for (int m = 1; m <= L; ++m)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < n; ++i) {
        const int64_t r = (2 * e + s) * (int64_t)(2 * n * A);
        v[m][s][i] = ym[m][r + i * A + a];
        u[m][s][i] = ym[m][r + n * A + i * A + a];
        go[m][s][i] = gom[m][(2 * e + s) * (n * A) + i * A + a];
      }
  // gate: out = u (1 + g) + ...
#pragma unroll
  for (int m = 0; m <= L; ++m)
#pragma unroll
    for (int i = 0; i < n; ++i) {
      const T z = y0[r0 + cg + (m * n + i) * A + a];
      const T sg = T(1) / (T(1) + exp(-z));
      const T g = T(TACE_ACE_SCST) * sg;
      T gz = go[m][0][i] * u[m][0][i];
      gu[m][0][i] = go[m][0][i] * (T(1) + g);
      gv[m][0][i] = gv[m][1][i] = T(0);
      if (m > 0) {
        gz += go[m][1][i] * u[m][1][i];
        gu[m][1][i] = go[m][1][i] * (T(1) + g);
      } else {
        gu[m][1][i] = T(0);
      }
      gy0[r0 + cg + (m * n + i) * A + a] = out_cvt<TO>(gz * T(TACE_ACE_SCST) * sg * (T(1) - sg));
    }
  int p = 0;
#pragma unroll
  for (int m3 = 0; m3 <= L; ++m3) {
    const T sc = T(1) / sqrt(T(AcePaths<L>::count(m3)));
#pragma unroll
    for (int m1 = 0; m1 <= L; ++m1)
#pragma unroll
      for (int m2 = 0; m2 <= m1; ++m2) {
        const bool sum = m1 + m2 == m3;
        if (!sum && m1 - m2 != m3) continue;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          const T zc = y0[r0 + (p * n + i) * A + a];
          const T sg = T(1) / (T(1) + exp(-zc));
          const T w = T(TACE_ACE_SCST) * sg;
          const T ar = u[m1][0][i], ai = u[m1][1][i], br = v[m2][0][i], bi = v[m2][1][i];
          T zr, zi;
          if (sum) { zr = ar * br - ai * bi; zi = ar * bi + ai * br; }
          else { zr = ar * br + ai * bi; zi = ai * br - ar * bi; }
          const T Gre = go[m3][0][i] * sc, Gim = m3 > 0 ? go[m3][1][i] * sc : T(0);
          gy0[r0 + (p * n + i) * A + a] = out_cvt<TO>((Gre * zr + Gim * zi) * T(TACE_ACE_SCST) * sg * (T(1) - sg));
          const T Gr = Gre * w, Gi = Gim * w;
          if (sum) {
            gu[m1][0][i] += Gr * br + Gi * bi;
            gu[m1][1][i] += Gi * br - Gr * bi;
            gv[m2][0][i] += Gr * ar + Gi * ai;
            gv[m2][1][i] += Gi * ar - Gr * ai;
          } else {
            gu[m1][0][i] += Gr * br - Gi * bi;
            gu[m1][1][i] += Gr * bi + Gi * br;
            gv[m2][0][i] += Gr * ar + Gi * ai;
            gv[m2][1][i] += Gr * ai - Gi * ar;
          }
        }
        ++p;
      }
  }
#pragma unroll
  for (int i = 0; i < n; ++i) {
    gy0[r0 + cu0 + i * A + a] = out_cvt<TO>(gu[0][0][i]);
    gy0[r0 + cv0 + i * A + a] = out_cvt<TO>(gv[0][0][i]);
  }
#pragma unroll
  for (int m = 1; m <= L; ++m)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < n; ++i) {
        const int64_t r = (2 * e + s) * (int64_t)(2 * n * A);
        gym[m][r + i * A + a] = out_cvt<TO>(gv[m][s][i]);
        gym[m][r + n * A + i * A + a] = out_cvt<TO>(gu[m][s][i]);
      }
}

// ------------------------------------------------------------ graph softmax --
// alpha[e,h] = exp(s - max_n) / (sum_{in-edges of n} exp(s - max_n) + 1e-16),
// n = receiver of e; one thread per (receiver, head), edges in CSR order.
template <typename T>
__global__ __launch_bounds__(256) void k_softmax_fwd(const T* __restrict__ s, const int* __restrict__ rowptr,
                                                     const int* __restrict__ eid, int N, int H,
                                                     T* __restrict__ alpha) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)N * H) return;
  const int n = (int)(t / H), h = (int)(t - (int64_t)n * H);
  const int b = rowptr[n], e = rowptr[n + 1];
  T mx = -INFINITY;
  for (int i = b; i < e; ++i) mx = fmax(mx, s[(int64_t)(eid ? eid[i] : i) * H + h]);
  T sum = 0;
  for (int i = b; i < e; ++i) sum += exp(s[(int64_t)(eid ? eid[i] : i) * H + h] - mx);
  const T inv = T(1) / (sum + T(1e-16));
  for (int i = b; i < e; ++i) {
    const int64_t j = (int64_t)(eid ? eid[i] : i) * H + h;
    alpha[j] = exp(s[j] - mx) * inv;
  }
}

// grad_s = alpha * (grad_alpha - sum_{in-edges} alpha grad_alpha)
template <typename T>
__global__ __launch_bounds__(256) void k_softmax_bwd(const T* __restrict__ alpha, const T* __restrict__ ga,
                                                     const int* __restrict__ rowptr, const int* __restrict__ eid,
                                                     int N, int H, T* __restrict__ gs) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)N * H) return;
  const int n = (int)(t / H), h = (int)(t - (int64_t)n * H);
  const int b = rowptr[n], e = rowptr[n + 1];
  T dot = 0;
  for (int i = b; i < e; ++i) {
    const int64_t j = (int64_t)(eid ? eid[i] : i) * H + h;
    dot += alpha[j] * ga[j];
  }
  for (int i = b; i < e; ++i) {
    const int64_t j = (int64_t)(eid ? eid[i] : i) * H + h;
    gs[j] = alpha[j] * (ga[j] - dot);
  }
}

// --------------------------------------------------- rotate out + scatter --
// out[n, k, c] = sum_{e -> n} sum_r W[e, r, k] alpha[e, c / Ch] m[e, r, c]
// written group-major (block l of the batch = [N, 2l+1, C] at N*C*l^2) at
// feature row map[n].  One workgroup per receiver, one lane per channel.
template <typename T, int L>
__global__ __launch_bounds__(512) void k_rotout_fwd(const Blk<const T> m, const T* __restrict__ alpha,
                                                    const T* __restrict__ W, const int* __restrict__ rowptr,
                                                    const int* __restrict__ eid, const int* __restrict__ map,
                                                    int N, int C, int H, T* __restrict__ out) {
  constexpr int K = (L + 1) * (L + 1);
  const int n0 = blockIdx.x;
  const int c = threadIdx.x;
  if (n0 >= N || c >= C) return;
  const int Ch = C / H, h = c / Ch;
  T acc[K];
#pragma unroll
  for (int k = 0; k < K; ++k) acc[k] = 0;
  for (int i = rowptr[n0]; i < rowptr[n0 + 1]; ++i) {
    const int64_t e = eid ? eid[i] : i;
    const T a = alpha[e * H + h];
    const T* w = W + e * K * K;
    T v[K];
#pragma unroll
    for (int r = 0; r < K; ++r) v[r] = a * erow<L>(m, e, r, C)[c];
#pragma unroll
    for (int r = 0; r < K; ++r)
#pragma unroll
      for (int k = 0; k < K; ++k) acc[k] += w[r * K + k] * v[r];
  }
  const int n = map ? map[n0] : n0;
  const int64_t NN = N;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    int l = 0;
    while ((l + 1) * (l + 1) <= k) ++l;
    const int j = k - l * l;
    out[NN * C * l * l + ((int64_t)n * (2 * l + 1) + j) * C + c] = acc[k];
  }
}

// backward, one wavefront per edge (n = map[dst[e]] or dst[e]):
//   t[r] = sum_k W[e,r,k] g[n,k,c];  g_m[e,r,c] = alpha[e,h(c)] t[r];
//   g_alpha[e,h] = sum over the head's channels and rows of m[e,r,c] t[r];
//   g_W[e,r,k] = sum_c alpha[e,h(c)] m[e,r,c] g[n,k,c].
template <typename T, typename TO, int L, int NS>
__global__ __launch_bounds__(256) void k_rotout_bwd(const Blk<const T> m, const T* __restrict__ alpha,
                                                    const T* __restrict__ W, const T* __restrict__ gout,
                                                    const int64_t* __restrict__ dst, const int* __restrict__ map,
                                                    int N, int64_t E, int C, int H, const Blk<TO> gm,
                                                    T* __restrict__ galpha, T* __restrict__ gW) {
  constexpr int K = (L + 1) * (L + 1), P = (K * K + 15) / 16 * 16;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const int Ch = C / H;
  const int64_t n0 = dst[e];
  const bool okn = n0 >= 0 && n0 < N;
  const int64_t n = okn ? (map ? (int64_t)map[n0] : n0) : 0;
  const int64_t NN = N;
  const T* w = W + e * K * K;
  T p[P];
#pragma unroll
  for (int i = 0; i < P; ++i) p[i] = T(0);
  T run[1] = {T(0)};
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j >= C) break;
    const int c = lane + 64 * j;
    const bool act = c < C;
    const int h = act ? c / Ch : 0;
    const T a = alpha[e * H + h];
    T g[K];
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      int l = 0;
      while ((l + 1) * (l + 1) <= kk) ++l;
      const int jj = kk - l * l;
      g[kk] = act && okn ? gout[NN * C * l * l + (n * (2 * l + 1) + jj) * C + c] : T(0);
    }
    T v[1] = {T(0)};
    if (act) {
#pragma unroll
      for (int r = 0; r < K; ++r) {
        T t = 0;
#pragma unroll
        for (int kk = 0; kk < K; ++kk) t += w[r * K + kk] * g[kk];
        const T mv = erow<L>(m, e, r, C)[c];
        erow<L>(gm, e, r, C)[c] = out_cvt<TO>(a * t);
        v[0] += mv * t;
        const T am = a * mv;
#pragma unroll
        for (int kk = 0; kk < K; ++kk) p[r * K + kk] += am * g[kk];
      }
    }
    if (head_sum<T, 1>(v, run, j, Ch, lane) && act) galpha[e * H + h] = v[0];
  }
  store_lane_sums<T, P>(p, K * K, gW + e * K * K, lane);
}

// ------------------------------------------------------------------ C ABI --
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

extern "C" {

int tace_edge_wigner_fwd(int dtype, const void* vec, int64_t n_edges, int32_t lmax, void* wigner, void* stream) {
  if (n_edges < 0 || lmax < 1 || lmax > 3) return tace_fail_msg("tace_edge_wigner_fwd: lmax must be 1..3");
  if (n_edges == 0) return 0;
  if (!vec || !wigner) return tace_fail_msg("tace_edge_wigner_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges + 63) / 64)), b(64);
#define WIG_F(TT, LL) hipLaunchKernelGGL((k_wigner_fwd<TT, LL>), g, b, 0, s, (const TT*)vec, n_edges, (TT*)wigner)
  if (dtype == TACE_F32) {
    if (lmax == 1) WIG_F(float, 1); else if (lmax == 2) WIG_F(float, 2); else WIG_F(float, 3);
  } else if (dtype == TACE_F64) {
    if (lmax == 1) WIG_F(double, 1); else if (lmax == 2) WIG_F(double, 2); else WIG_F(double, 3);
  } else {
    return tace_fail_msg("tace_edge_wigner_fwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef WIG_F
  return tace_check_launch("tace_edge_wigner_fwd");
}

int tace_edge_wigner_bwd(int dtype, const void* vec, const void* g_wigner, int64_t n_edges, int32_t lmax,
                         void* g_vec, void* stream) {
  if (n_edges < 0 || lmax < 1 || lmax > 3) return tace_fail_msg("tace_edge_wigner_bwd: lmax must be 1..3");
  if (n_edges == 0) return 0;
  if (!vec || !g_wigner || !g_vec) return tace_fail_msg("tace_edge_wigner_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges + 63) / 64)), b(64);
#define WIG_B(TT, LL) \
  hipLaunchKernelGGL((k_wigner_bwd<TT, LL>), g, b, 0, s, (const TT*)vec, (const TT*)g_wigner, n_edges, (TT*)g_vec)
  if (dtype == TACE_F32) {
    if (lmax == 1) WIG_B(float, 1); else if (lmax == 2) WIG_B(float, 2); else WIG_B(float, 3);
  } else if (dtype == TACE_F64) {
    if (lmax == 1) WIG_B(double, 1); else if (lmax == 2) WIG_B(double, 2); else WIG_B(double, 3);
  } else {
    return tace_fail_msg("tace_edge_wigner_bwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef WIG_B
  return tace_check_launch("tace_edge_wigner_bwd");
}

static int score_checks(const char* who, int64_t E, int32_t lmax, int32_t C, int32_t H) {
  char msg[160];
  if (E < 0 || lmax < 1 || lmax > 3 || C <= 0 || C > TACE_MAX_CHANNELS || H <= 0 || C % H ||
      (C / H < 64 ? 64 % (C / H) : (C / H) % 64)) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (lmax 1..3, channels <= %d, divisible by heads; per-head width a "
             "divisor or a multiple of 64)", who, TACE_MAX_CHANNELS);
    return tace_fail_msg(msg);
  }
  return 0;
}

static dim3 wave_grid(int64_t E) { return dim3((unsigned)((E + 3) / 4)); }

int tace_tece_score_fwd(int dtype, const void* const* q, const void* const* k, const void* radial_proj,
                        const void* tscale, int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads,
                        void* score, void* stream) {
  if (score_checks("tace_tece_score_fwd", n_edges, lmax, channels, heads)) return -1;
  if (n_edges == 0) return 0;
  if (!blocks_ok(q, lmax) || !blocks_ok(k, lmax) || !radial_proj || !tscale || !score)
    return tace_fail_msg("tace_tece_score_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
#define SC_F(TT, LL)                                                                                            \
  TACE_SLOTS_DISPATCH(channels, NS,                                                                             \
    hipLaunchKernelGGL((k_score_fwd<TT, LL, NS>), g, b, 0, s, blocks_of<const TT>(q, lmax),                 \
                       blocks_of<const TT>(k, lmax), (const TT*)radial_proj, (const TT*)tscale, n_edges, channels, \
                       heads, (TT*)score))
  if (dtype == TACE_F32) {
    if (lmax == 1) { SC_F(float, 1) } else if (lmax == 2) { SC_F(float, 2) } else { SC_F(float, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { SC_F(double, 1) } else if (lmax == 2) { SC_F(double, 2) } else { SC_F(double, 3) }
  } else {
    return tace_fail_msg("tace_tece_score_fwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef SC_F
  return tace_check_launch("tace_tece_score_fwd");
}

int tace_tece_score_bwd(int dtype, const void* const* q, const void* const* k, const void* radial_proj,
                        const void* tscale, const void* g_score, int64_t n_edges, int32_t lmax, int32_t channels,
                        int32_t heads, const void* const* g_q, const void* const* g_k, void* g_radial_proj,
                        void* stream) {
  if (score_checks("tace_tece_score_bwd", n_edges, lmax, channels, heads)) return -1;
  if (n_edges == 0) return 0;
  if (!blocks_ok(q, lmax) || !blocks_ok(k, lmax) || !radial_proj || !tscale || !g_score || !blocks_ok(g_q, lmax) ||
      !blocks_ok(g_k, lmax) || !g_radial_proj)
    return tace_fail_msg("tace_tece_score_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
#define SC_B(TT, TO, LL)                                                                                        \
  TACE_SLOTS_DISPATCH(channels, NS,                                                                             \
    hipLaunchKernelGGL((k_score_bwd<TT, TO, LL, NS>), g, b, 0, s, blocks_of<const TT>(q, lmax),             \
                       blocks_of<const TT>(k, lmax), (const TT*)radial_proj, (const TT*)tscale,              \
                       (const TT*)g_score, n_edges, channels, heads, blocks_of<TO>(g_q, lmax),               \
                       blocks_of<TO>(g_k, lmax), (TT*)g_radial_proj))
  if (dtype == TACE_F32) {
    if (lmax == 1) { SC_B(float, float, 1) } else if (lmax == 2) { SC_B(float, float, 2) } else { SC_B(float, float, 3) }
  } else if (dtype == TACE_F32_BF16) {
    if (lmax == 1) { SC_B(float, bf16_t, 1) } else if (lmax == 2) { SC_B(float, bf16_t, 2) } else { SC_B(float, bf16_t, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { SC_B(double, double, 1) } else if (lmax == 2) { SC_B(double, double, 2) } else { SC_B(double, double, 3) }
  } else {
    return tace_fail_msg("tace_tece_score_bwd: dtype must be TACE_F32, TACE_F32_BF16 or TACE_F64");
  }
#undef SC_B
  return tace_check_launch("tace_tece_score_bwd");
}

static int rotin_checks(const char* who, int64_t n_rows, int64_t E, int32_t lmax, int32_t C) {
  char msg[128];
  if (n_rows < 0 || E < 0 || lmax < 1 || lmax > 3 || C <= 0 || C > TACE_MAX_CHANNELS) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (lmax 1..3, channels 1..%d)", who, TACE_MAX_CHANNELS);
    return tace_fail_msg(msg);
  }
  return 0;
}

int tace_edge_rotate_in_fwd(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                            const int64_t* rows_dst, const void* radial_w, int64_t n_rows, int64_t n_edges,
                            int32_t lmax, int32_t channels, const void* const* m_src, const void* const* m_dst,
                            const void* const* m_w, void* stream) {
  if (rotin_checks("tace_edge_rotate_in_fwd", n_rows, n_edges, lmax, channels)) return -1;
  if (n_edges == 0) return 0;
  if (!x || !wigner || !rows_src || !rows_dst || !blocks_ok(m_src, lmax) || !blocks_ok(m_dst, lmax) ||
      (radial_w && !blocks_ok(m_w, lmax)))
    return tace_fail_msg("tace_edge_rotate_in_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
  // float32 features, even channel count, 8-byte aligned x / radial_w and
  // outputs aligned to two elements: two channels per lane
  const size_t oal = dtype == TACE_F32_BF16 ? 4 : 8;
  bool pairs = (dtype == TACE_F32 || dtype == TACE_F32_BF16) && (channels & 1) == 0 && channels <= 512 &&
               ((uintptr_t)x & 7) == 0 && ((uintptr_t)radial_w & 7) == 0;
  for (int m = 0; pairs && m <= lmax; ++m)
    pairs = ((uintptr_t)m_src[m] % oal) == 0 && ((uintptr_t)m_dst[m] % oal) == 0 &&
            (!radial_w || ((uintptr_t)m_w[m] % oal) == 0);
  if (pairs) {
#define RI_P(TO, LL)                                                                                          \
  TACE_SLOTS_DISPATCH(channels, NP,                                                                           \
    hipLaunchKernelGGL((k_rotin_fwd_pairs<TO, LL, NP>), g, b, 0, s, (const float*)x, (const float*)wigner,     \
                       rows_src, rows_dst, (const float*)radial_w, n_rows, n_edges, channels,                  \
                       blocks_of<TO>(m_src, lmax), blocks_of<TO>(m_dst, lmax),                                 \
                       blocks_of<TO>(radial_w ? m_w : nullptr, lmax)))
    if (dtype == TACE_F32) {
      if (lmax == 1) { RI_P(float, 1) } else if (lmax == 2) { RI_P(float, 2) } else { RI_P(float, 3) }
    } else {
      if (lmax == 1) { RI_P(bf16_t, 1) } else if (lmax == 2) { RI_P(bf16_t, 2) } else { RI_P(bf16_t, 3) }
    }
#undef RI_P
    return tace_check_launch("tace_edge_rotate_in_fwd");
  }
#define RI_F(TT, TO, LL)                                                                                    \
  TACE_SLOTS_DISPATCH(2 * channels, NS,                                                                     \
    hipLaunchKernelGGL((k_rotin_fwd<TT, TO, LL, NS>), g, b, 0, s, (const TT*)x, (const TT*)wigner, rows_src, \
                       rows_dst, (const TT*)radial_w, n_rows, n_edges, channels, blocks_of<TO>(m_src, lmax), \
                       blocks_of<TO>(m_dst, lmax), blocks_of<TO>(radial_w ? m_w : nullptr, lmax)))
  if (dtype == TACE_F32) {
    if (lmax == 1) { RI_F(float, float, 1) } else if (lmax == 2) { RI_F(float, float, 2) } else { RI_F(float, float, 3) }
  } else if (dtype == TACE_F32_BF16) {
    if (lmax == 1) { RI_F(float, bf16_t, 1) } else if (lmax == 2) { RI_F(float, bf16_t, 2) } else { RI_F(float, bf16_t, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { RI_F(double, double, 1) } else if (lmax == 2) { RI_F(double, double, 2) } else { RI_F(double, double, 3) }
  } else {
    return tace_fail_msg("tace_edge_rotate_in_fwd: dtype must be TACE_F32, TACE_F32_BF16 or TACE_F64");
  }
#undef RI_F
  return tace_check_launch("tace_edge_rotate_in_fwd");
}

int tace_edge_rotate_in_bwd(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                            const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                            const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows, int64_t n_edges,
                            int32_t lmax, int32_t channels, void* g_x_src, void* g_x_dst, void* g_wigner,
                            void* g_radial_w, void* stream) {
  if (rotin_checks("tace_edge_rotate_in_bwd", n_rows, n_edges, lmax, channels)) return -1;
  if (n_edges == 0) return 0;
  if (!x || !wigner || !rows_src || !rows_dst || !g_x_src || !g_x_dst || !g_wigner || (g_m_w && !radial_w))
    return tace_fail_msg("tace_edge_rotate_in_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
#define RI_B(TT, LL)                                                                                          \
  TACE_SLOTS_DISPATCH(2 * channels, NS,                                                                       \
    hipLaunchKernelGGL((k_rotin_bwd<TT, LL, NS, false>), g, b, 0, s, (const TT*)x, (const TT*)wigner, rows_src,     \
                       rows_dst, (const TT*)radial_w, blocks_of<const TT>(g_m_src, lmax),                   \
                       blocks_of<const TT>(g_m_dst, lmax), blocks_of<const TT>(g_m_w, lmax), n_rows, n_edges,  \
                       channels, (TT*)g_x_src, (TT*)g_x_dst, (TT*)g_wigner, (TT*)g_radial_w))
  if (dtype == TACE_F32) {
    if (lmax == 1) { RI_B(float, 1) } else if (lmax == 2) { RI_B(float, 2) } else { RI_B(float, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { RI_B(double, 1) } else if (lmax == 2) { RI_B(double, 2) } else { RI_B(double, 3) }
  } else {
    return tace_fail_msg("tace_edge_rotate_in_bwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef RI_B
  return tace_check_launch("tace_edge_rotate_in_bwd");
}

int tace_edge_rotate_in_bwd_runs(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                                 const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                                 const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows,
                                 int64_t n_edges, int32_t lmax, int32_t channels, void* g_x_src, void* g_x_dst_runs,
                                 void* g_wigner, void* g_radial_w, void* stream) {
  if (rotin_checks("tace_edge_rotate_in_bwd_runs", n_rows, n_edges, lmax, channels)) return -1;
  const size_t es = dtype == TACE_F64 ? 8 : 4;
  const size_t lds = (size_t)4 * (lmax + 1) * (lmax + 1) * channels * es;
  if (lds > 65536) return tace_fail_msg("tace_edge_rotate_in_bwd_runs: 4 (lmax+1)^2 channels values exceed 64 KB of LDS");
  if (n_edges == 0) return 0;
  if (!x || !wigner || !rows_src || !rows_dst || !g_x_src || !g_x_dst_runs || !g_wigner || (g_m_w && !radial_w))
    return tace_fail_msg("tace_edge_rotate_in_bwd_runs: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
#define RI_BR(TT, LL)                                                                                            \
  TACE_SLOTS_DISPATCH(2 * channels, NS,                                                                         \
    hipLaunchKernelGGL((k_rotin_bwd<TT, LL, NS, true>), g, b, lds, s, (const TT*)x, (const TT*)wigner, rows_src, \
                       rows_dst, (const TT*)radial_w, blocks_of<const TT>(g_m_src, lmax),                     \
                       blocks_of<const TT>(g_m_dst, lmax), blocks_of<const TT>(g_m_w, lmax), n_rows, n_edges,    \
                       channels, (TT*)g_x_src, (TT*)g_x_dst_runs, (TT*)g_wigner, (TT*)g_radial_w))
  if (dtype == TACE_F32) {
    if (lmax == 1) { RI_BR(float, 1) } else if (lmax == 2) { RI_BR(float, 2) } else { RI_BR(float, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { RI_BR(double, 1) } else if (lmax == 2) { RI_BR(double, 2) } else { RI_BR(double, 3) }
  } else {
    return tace_fail_msg("tace_edge_rotate_in_bwd_runs: dtype must be TACE_F32 or TACE_F64");
  }
#undef RI_BR
  return tace_check_launch("tace_edge_rotate_in_bwd_runs");
}

int tace_graph_softmax_fwd(int dtype, const void* score, const int32_t* rowptr, const int32_t* eid, int64_t n_nodes,
                           int32_t heads, void* alpha, void* stream) {
  if (n_nodes < 0 || n_nodes > INT32_MAX || heads <= 0) return tace_fail_msg("tace_graph_softmax_fwd: bad sizes");
  if (n_nodes == 0) return 0;
  if (!rowptr) return tace_fail_msg("tace_graph_softmax_fwd: null rowptr");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_nodes * heads + 255) / 256)), b(256);
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_softmax_fwd<float>, g, b, 0, s, (const float*)score, rowptr, eid, (int)n_nodes, heads,
                       (float*)alpha);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_softmax_fwd<double>, g, b, 0, s, (const double*)score, rowptr, eid, (int)n_nodes, heads,
                       (double*)alpha);
  else
    return tace_fail_msg("tace_graph_softmax_fwd: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_graph_softmax_fwd");
}

int tace_graph_softmax_bwd(int dtype, const void* alpha, const void* g_alpha, const int32_t* rowptr,
                           const int32_t* eid, int64_t n_nodes, int32_t heads, void* g_score, void* stream) {
  if (n_nodes < 0 || n_nodes > INT32_MAX || heads <= 0) return tace_fail_msg("tace_graph_softmax_bwd: bad sizes");
  if (n_nodes == 0) return 0;
  if (!rowptr) return tace_fail_msg("tace_graph_softmax_bwd: null rowptr");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_nodes * heads + 255) / 256)), b(256);
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_softmax_bwd<float>, g, b, 0, s, (const float*)alpha, (const float*)g_alpha, rowptr, eid,
                       (int)n_nodes, heads, (float*)g_score);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_softmax_bwd<double>, g, b, 0, s, (const double*)alpha, (const double*)g_alpha, rowptr,
                       eid, (int)n_nodes, heads, (double*)g_score);
  else
    return tace_fail_msg("tace_graph_softmax_bwd: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_graph_softmax_bwd");
}

static int rotout_checks(const char* who, int64_t N, int32_t lmax, int32_t C, int32_t H) {
  char msg[160];
  if (N < 0 || N > INT32_MAX || lmax < 1 || lmax > 3 || C <= 0 || C > TACE_MAX_CHANNELS || H <= 0 || C % H ||
      (C / H > 64 && (C / H) % 64)) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (lmax 1..3, channels <= %d, divisible by heads; per-head width a "
             "divisor or a multiple of 64)", who, TACE_MAX_CHANNELS);
    return tace_fail_msg(msg);
  }
  return 0;
}

int tace_tece_rotate_out_fwd(int dtype, const void* const* m, const void* alpha, const void* wigner,
                             const int32_t* rowptr,
                             const int32_t* eid, const int32_t* node_map, int64_t n_nodes, int32_t lmax,
                             int32_t channels, int32_t heads, void* out, void* stream) {
  if (rotout_checks("tace_tece_rotate_out_fwd", n_nodes, lmax, channels, heads)) return -1;
  if (n_nodes == 0) return 0;
  if (!rowptr || !out) return tace_fail_msg("tace_tece_rotate_out_fwd: null pointer");
  if (!m) return tace_fail_msg("tace_tece_rotate_out_fwd: null block array");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)n_nodes), b((unsigned)((channels + 63) / 64 * 64));
#define ROT_F(TT, LL)                                                                                           \
  hipLaunchKernelGGL((k_rotout_fwd<TT, LL>), g, b, 0, s, blocks_of<const TT>(m, lmax), (const TT*)alpha,      \
                     (const TT*)wigner, rowptr, eid, node_map, (int)n_nodes, channels, heads, (TT*)out)
  if (dtype == TACE_F32) {
    if (lmax == 1) ROT_F(float, 1); else if (lmax == 2) ROT_F(float, 2); else ROT_F(float, 3);
  } else if (dtype == TACE_F64) {
    if (lmax == 1) ROT_F(double, 1); else if (lmax == 2) ROT_F(double, 2); else ROT_F(double, 3);
  } else {
    return tace_fail_msg("tace_tece_rotate_out_fwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef ROT_F
  return tace_check_launch("tace_tece_rotate_out_fwd");
}

int tace_tece_rotate_out_bwd(int dtype, const void* const* m, const void* alpha, const void* wigner,
                             const void* g_out, const int64_t* dst, const int32_t* node_map, int64_t n_nodes,
                             int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads, const void* const* g_m,
                             void* g_alpha, void* g_wigner, void* stream) {
  if (rotout_checks("tace_tece_rotate_out_bwd", n_nodes, lmax, channels, heads)) return -1;
  if (n_edges < 0) return tace_fail_msg("tace_tece_rotate_out_bwd: negative edge count");
  if (n_edges == 0) return 0;
  if (!blocks_ok(m, lmax) || !alpha || !wigner || !g_out || !dst || !blocks_ok(g_m, lmax) || !g_alpha || !g_wigner)
    return tace_fail_msg("tace_tece_rotate_out_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
#define ROT_B(TT, TO, LL)                                                                                      \
  TACE_SLOTS_DISPATCH(channels, NS,                                                                            \
    hipLaunchKernelGGL((k_rotout_bwd<TT, TO, LL, NS>), g, b, 0, s, blocks_of<const TT>(m, lmax),             \
                       (const TT*)alpha, (const TT*)wigner, (const TT*)g_out, dst, node_map, (int)n_nodes,    \
                       n_edges, channels, heads, blocks_of<TO>(g_m, lmax), (TT*)g_alpha, (TT*)g_wigner))
  if (dtype == TACE_F32) {
    if (lmax == 1) { ROT_B(float, float, 1) } else if (lmax == 2) { ROT_B(float, float, 2) } else { ROT_B(float, float, 3) }
  } else if (dtype == TACE_F32_BF16) {
    if (lmax == 1) { ROT_B(float, bf16_t, 1) } else if (lmax == 2) { ROT_B(float, bf16_t, 2) } else { ROT_B(float, bf16_t, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { ROT_B(double, double, 1) } else if (lmax == 2) { ROT_B(double, double, 2) } else { ROT_B(double, double, 3) }
  } else {
    return tace_fail_msg("tace_tece_rotate_out_bwd: dtype must be TACE_F32, TACE_F32_BF16 or TACE_F64");
  }
#undef ROT_B
  return tace_check_launch("tace_tece_rotate_out_bwd");
}

int tace_tece_edge_ace_fwd(int dtype, const void* y0, const void* y1, const void* y2, const void* y3,
                           int64_t n_edges, int32_t lmax, int32_t hidden, void* o0, void* o1, void* o2, void* o3,
                           void* stream) {
  if (n_edges < 0 || lmax < 1 || lmax > 3 || hidden <= 0)
    return tace_fail_msg("tace_tece_edge_ace_fwd: bad sizes (lmax 1..3)");
  if (n_edges == 0) return 0;
  const void* ys[4] = {y0, y1, y2, y3};
  void* os[4] = {o0, o1, o2, o3};
  for (int m = 0; m <= lmax; ++m)
    if (!ys[m] || !os[m]) return tace_fail_msg("tace_tece_edge_ace_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges * hidden + 255) / 256)), b(256);
#define ACE_F(TT, TO, LL)                                                                                       \
  hipLaunchKernelGGL((k_edge_ace_fwd<TT, TO, LL>), g, b, 0, s, (const TT*)y0, (const TT*)y1, (const TT*)y2,    \
                     (const TT*)y3, n_edges, hidden, (TO*)o0, (TO*)o1, (TO*)o2, (TO*)o3)
  if (dtype == TACE_F32) {
    if (lmax == 1) ACE_F(float, float, 1); else if (lmax == 2) ACE_F(float, float, 2); else ACE_F(float, float, 3);
  } else if (dtype == TACE_F32_BF16) {
    if (lmax == 1) ACE_F(float, bf16_t, 1); else if (lmax == 2) ACE_F(float, bf16_t, 2); else ACE_F(float, bf16_t, 3);
  } else if (dtype == TACE_F64) {
    if (lmax == 1) ACE_F(double, double, 1); else if (lmax == 2) ACE_F(double, double, 2); else ACE_F(double, double, 3);
  } else {
    return tace_fail_msg("tace_tece_edge_ace_fwd: dtype must be TACE_F32, TACE_F32_BF16 or TACE_F64");
  }
#undef ACE_F
  return tace_check_launch("tace_tece_edge_ace_fwd");
}

int tace_tece_edge_ace_bwd(int dtype, const void* y0, const void* y1, const void* y2, const void* y3,
                           const void* g_o0, const void* g_o1, const void* g_o2, const void* g_o3, int64_t n_edges,
                           int32_t lmax, int32_t hidden, void* g_y0, void* g_y1, void* g_y2, void* g_y3,
                           void* stream) {
  if (n_edges < 0 || lmax < 1 || lmax > 3 || hidden <= 0)
    return tace_fail_msg("tace_tece_edge_ace_bwd: bad sizes (lmax 1..3)");
  if (n_edges == 0) return 0;
  const void* ys[4] = {y0, y1, y2, y3};
  const void* gos[4] = {g_o0, g_o1, g_o2, g_o3};
  void* gys[4] = {g_y0, g_y1, g_y2, g_y3};
  for (int m = 0; m <= lmax; ++m)
    if (!ys[m] || !gos[m] || !gys[m]) return tace_fail_msg("tace_tece_edge_ace_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges * hidden + 255) / 256)), b(256);
#define ACE_B(TT, TO, LL)                                                                                       \
  hipLaunchKernelGGL((k_edge_ace_bwd<TT, TO, LL>), g, b, 0, s, (const TT*)y0, (const TT*)y1, (const TT*)y2,    \
                     (const TT*)y3, (const TT*)g_o0, (const TT*)g_o1, (const TT*)g_o2, (const TT*)g_o3, n_edges, \
                     hidden, (TO*)g_y0, (TO*)g_y1, (TO*)g_y2, (TO*)g_y3)
  if (dtype == TACE_F32) {
    if (lmax == 1) ACE_B(float, float, 1); else if (lmax == 2) ACE_B(float, float, 2); else ACE_B(float, float, 3);
  } else if (dtype == TACE_F32_BF16) {
    if (lmax == 1) ACE_B(float, bf16_t, 1); else if (lmax == 2) ACE_B(float, bf16_t, 2); else ACE_B(float, bf16_t, 3);
  } else if (dtype == TACE_F64) {
    if (lmax == 1) ACE_B(double, double, 1); else if (lmax == 2) ACE_B(double, double, 2); else ACE_B(double, double, 3);
  } else {
    return tace_fail_msg("tace_tece_edge_ace_bwd: dtype must be TACE_F32, TACE_F32_BF16 or TACE_F64");
  }
#undef ACE_B
  return tace_check_launch("tace_tece_edge_ace_bwd");
}

}  // extern "C"
