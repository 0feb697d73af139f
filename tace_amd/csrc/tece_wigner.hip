// MI355X (gfx950) edge-frame Wigner matrices of the TECE convolution in the
// SO(2) m layout from the edge vector (tace/models/o2/rotation_matrix.py:74-88,
// tace/models/o2/wigner.py:231-357), forward and the exact backward to the edge
// vector (reverse mode through the D^l recursion, dual numbers for the frame).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"
#include "tece_common.h"
#include "gen/wigner.inc"

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

}  // extern "C"
