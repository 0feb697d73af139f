// MI355X (gfx950) kernels of the TECE radial-rotary edge attention
// (tace/models/_e3nn/archive/oam_2026_07_05.py:547-823):
//   * edge-frame Wigner matrices in the SO(2) "m layout" from the edge vector
//     (tace/models/o2/rotation_matrix.py:74-88, tace/models/o2/wigner.py:231-357),
//     forward and the exact backward to the edge vector (dual numbers);
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

template <typename T, int L>
__global__ __launch_bounds__(64) void k_wigner_fwd(const T* __restrict__ vec, int64_t E, T* __restrict__ W) {
  constexpr int K = (L + 1) * (L + 1);
  const int64_t e = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (e >= E) return;
  T w[K * K];
  wigner_m<T, T, L>(vec[3 * e], vec[3 * e + 1], vec[3 * e + 2], w);
  T* o = W + e * K * K;
#pragma unroll
  for (int i = 0; i < K * K; ++i) o[i] = w[i];
}

template <typename T, int L>
__global__ __launch_bounds__(64) void k_wigner_bwd(const T* __restrict__ vec, const T* __restrict__ gW, int64_t E,
                                                   T* __restrict__ gv) {
  constexpr int K = (L + 1) * (L + 1);
  const int64_t e = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (e >= E) return;
  Dual3<T> x(vec[3 * e]), y(vec[3 * e + 1]), z(vec[3 * e + 2]);
  x.d[0] = T(1); y.d[1] = T(1); z.d[2] = T(1);
  Dual3<T> w[K * K];
  wigner_m<T, Dual3<T>, L>(x, y, z, w);
  const T* g = gW + e * K * K;
  T a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
  for (int i = 0; i < K * K; ++i) {
    const T gi = g[i];
    a0 += gi * w[i].d[0]; a1 += gi * w[i].d[1]; a2 += gi * w[i].d[2];
  }
  gv[3 * e] = a0; gv[3 * e + 1] = a1; gv[3 * e + 2] = a2;
}

// -------------------------------------------------------------- QK score --
// score[e,h] = (S0 + sum_m cos(m phi) A_m + sin(m phi) B_m) * tscale[h] + rp[e,h],
// phi = pi tanh(rp[e, H+h]);  S0 = sum over the m = 0 rows of q.k,
// A_m = sum(q_re k_re + q_im k_im), B_m = sum(q_im k_re - q_re k_im) over the
// +-m rows and the head's Ch channels.  One thread per (edge, head).
template <typename T>
__device__ __forceinline__ void rows_of_m(int L, int m, int* re, int* n) {
  int off = L + 1;
  for (int mm = 1; mm < m; ++mm) off += 2 * (L + 1 - mm);
  *re = off;
  *n = L + 1 - m;
}

template <typename T>
__global__ __launch_bounds__(256) void k_score_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ rp, const T* __restrict__ tscale,
                                                   int64_t E, int L, int C, int H, T* __restrict__ score) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= E * H) return;
  const int64_t e = t / H;
  const int h = (int)(t - e * H);
  const int Ch = C / H, K = (L + 1) * (L + 1);
  const T* qe = q + e * K * C + h * Ch;
  const T* ke = k + e * K * C + h * Ch;
  T s = 0;
  for (int r = 0; r <= L; ++r)
    for (int c = 0; c < Ch; ++c) s += qe[r * C + c] * ke[r * C + c];
  const T phi = T(M_PI) * tanh(rp[e * 2 * H + H + h]);
  for (int m = 1; m <= L; ++m) {
    int re, n;
    rows_of_m<T>(L, m, &re, &n);
    T A = 0, B = 0;
    for (int j = 0; j < n; ++j)
      for (int c = 0; c < Ch; ++c) {
        const T qr = qe[(re + j) * C + c], qi = qe[(re + n + j) * C + c];
        const T kr = ke[(re + j) * C + c], ki = ke[(re + n + j) * C + c];
        A += qr * kr + qi * ki;
        B += qi * kr - qr * ki;
      }
    s += cos(m * phi) * A + sin(m * phi) * B;
  }
  score[t] = s * tscale[h] + rp[e * 2 * H + h];
}

template <typename T>
__global__ __launch_bounds__(256) void k_score_bwd(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ rp, const T* __restrict__ tscale,
                                                   const T* __restrict__ gs, int64_t E, int L, int C, int H,
                                                   T* __restrict__ gq, T* __restrict__ gk, T* __restrict__ grp) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= E * H) return;
  const int64_t e = t / H;
  const int h = (int)(t - e * H);
  const int Ch = C / H, K = (L + 1) * (L + 1);
  const int64_t base = e * K * C + h * Ch;
  const T g = gs[t];
  const T G = g * tscale[h];
  for (int r = 0; r <= L; ++r)
    for (int c = 0; c < Ch; ++c) {
      const int64_t i = base + r * C + c;
      const T qv = q[i], kv = k[i];
      gq[i] = G * kv;
      gk[i] = G * qv;
    }
  const T th = tanh(rp[e * 2 * H + H + h]);
  const T phi = T(M_PI) * th;
  T dphi = 0;
  for (int m = 1; m <= L; ++m) {
    int re, n;
    rows_of_m<T>(L, m, &re, &n);
    const T cs = cos(m * phi), sn = sin(m * phi);
    T A = 0, B = 0;
    for (int j = 0; j < n; ++j)
      for (int c = 0; c < Ch; ++c) {
        const int64_t ir = base + (re + j) * C + c, ii = base + (re + n + j) * C + c;
        const T qr = q[ir], qi = q[ii], kr = k[ir], ki = k[ii];
        A += qr * kr + qi * ki;
        B += qi * kr - qr * ki;
        gq[ir] = G * (cs * kr - sn * ki);
        gq[ii] = G * (cs * ki + sn * kr);
        gk[ir] = G * (cs * qr + sn * qi);
        gk[ii] = G * (cs * qi - sn * qr);
      }
    dphi += T(m) * (cs * B - sn * A);
  }
  grp[e * 2 * H + h] = g;
  grp[e * 2 * H + H + h] = G * dphi * T(M_PI) * (T(1) - th * th);
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
__global__ __launch_bounds__(512) void k_rotout_fwd(const T* __restrict__ m, const T* __restrict__ alpha,
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
    const T* me = m + e * K * C + c;
    T v[K];
#pragma unroll
    for (int r = 0; r < K; ++r) v[r] = a * me[(int64_t)r * C];
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

// backward: t[r] = sum_k W[e,r,k] g[dst,k,c];  g_m[e,r,c] = alpha t[r];
// g_alpha[e,h] = sum over the head's channels and rows of m[e,r,c] t[r]
// (lane reduction over Ch = 16/32/64 lanes, fixed order).
template <typename T, int L>
__global__ __launch_bounds__(512) void k_rotout_bwd(const T* __restrict__ m, const T* __restrict__ alpha,
                                                    const T* __restrict__ W, const T* __restrict__ gout,
                                                    const int* __restrict__ rowptr, const int* __restrict__ eid,
                                                    const int* __restrict__ map, int N, int C, int H,
                                                    T* __restrict__ gm, T* __restrict__ galpha) {
  constexpr int K = (L + 1) * (L + 1);
  const int n0 = blockIdx.x;
  const int c = threadIdx.x;
  if (n0 >= N) return;
  const bool act = c < C;
  const int cc = act ? c : C - 1;
  const int Ch = C / H, h = cc / Ch;
  const int n = map ? map[n0] : n0;
  const int64_t NN = N;
  T g[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    int l = 0;
    while ((l + 1) * (l + 1) <= k) ++l;
    const int j = k - l * l;
    g[k] = act ? gout[NN * C * l * l + ((int64_t)n * (2 * l + 1) + j) * C + cc] : T(0);
  }
  for (int i = rowptr[n0]; i < rowptr[n0 + 1]; ++i) {
    const int64_t e = eid ? eid[i] : i;
    const T a = alpha[e * H + h];
    const T* w = W + e * K * K;
    const T* me = m + e * K * C + cc;
    T p = 0;
#pragma unroll
    for (int r = 0; r < K; ++r) {
      T t = 0;
#pragma unroll
      for (int k = 0; k < K; ++k) t += w[r * K + k] * g[k];
      if (act) gm[e * K * C + (int64_t)r * C + c] = a * t;
      p += me[(int64_t)r * C] * t;
    }
    // sum p over the Ch lanes of the head (Ch divides 64 or is a multiple of 64)
    const int width = Ch < 64 ? Ch : 64;
    for (int o = width >> 1; o > 0; o >>= 1) p += __shfl_xor(p, o, 64);
    if (Ch <= 64) {
      if ((c & (width - 1)) == 0 && act) galpha[e * H + h] = p;
    } else {
      // heads wider than a wavefront: partial sums of the head's wavefronts go
      // through LDS in a fixed order
      __shared__ T part[16];
      const int wv = c >> 6, nw = (C + 63) >> 6;
      __syncthreads();
      if ((c & 63) == 0) part[wv] = p;
      __syncthreads();
      if (act && (c % Ch) == 0) {
        T s = 0;
        for (int q = c >> 6; q < ((c + Ch) >> 6) && q < nw; ++q) s += part[q];
        galpha[e * H + h] = s;
      }
    }
  }
}

// ------------------------------------------------------------------ C ABI --
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
  char msg[128];
  if (E < 0 || lmax < 1 || lmax > 3 || C <= 0 || H <= 0 || C % H) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (lmax 1..3, channels divisible by heads)", who);
    return tace_fail_msg(msg);
  }
  return 0;
}

int tace_tece_score_fwd(int dtype, const void* q, const void* k, const void* radial_proj, const void* tscale,
                        int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads, void* score, void* stream) {
  if (score_checks("tace_tece_score_fwd", n_edges, lmax, channels, heads)) return -1;
  if (n_edges == 0) return 0;
  if (!q || !k || !radial_proj || !tscale || !score) return tace_fail_msg("tace_tece_score_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges * heads + 255) / 256)), b(256);
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_score_fwd<float>, g, b, 0, s, (const float*)q, (const float*)k, (const float*)radial_proj,
                       (const float*)tscale, n_edges, lmax, channels, heads, (float*)score);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_score_fwd<double>, g, b, 0, s, (const double*)q, (const double*)k,
                       (const double*)radial_proj, (const double*)tscale, n_edges, lmax, channels, heads,
                       (double*)score);
  else
    return tace_fail_msg("tace_tece_score_fwd: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_tece_score_fwd");
}

int tace_tece_score_bwd(int dtype, const void* q, const void* k, const void* radial_proj, const void* tscale,
                        const void* g_score, int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads,
                        void* g_q, void* g_k, void* g_radial_proj, void* stream) {
  if (score_checks("tace_tece_score_bwd", n_edges, lmax, channels, heads)) return -1;
  if (n_edges == 0) return 0;
  if (!q || !k || !radial_proj || !tscale || !g_score || !g_q || !g_k || !g_radial_proj)
    return tace_fail_msg("tace_tece_score_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges * heads + 255) / 256)), b(256);
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_score_bwd<float>, g, b, 0, s, (const float*)q, (const float*)k, (const float*)radial_proj,
                       (const float*)tscale, (const float*)g_score, n_edges, lmax, channels, heads, (float*)g_q,
                       (float*)g_k, (float*)g_radial_proj);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_score_bwd<double>, g, b, 0, s, (const double*)q, (const double*)k,
                       (const double*)radial_proj, (const double*)tscale, (const double*)g_score, n_edges, lmax,
                       channels, heads, (double*)g_q, (double*)g_k, (double*)g_radial_proj);
  else
    return tace_fail_msg("tace_tece_score_bwd: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_tece_score_bwd");
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

int tace_tece_rotate_out_fwd(int dtype, const void* m, const void* alpha, const void* wigner, const int32_t* rowptr,
                             const int32_t* eid, const int32_t* node_map, int64_t n_nodes, int32_t lmax,
                             int32_t channels, int32_t heads, void* out, void* stream) {
  if (rotout_checks("tace_tece_rotate_out_fwd", n_nodes, lmax, channels, heads)) return -1;
  if (n_nodes == 0) return 0;
  if (!rowptr || !out) return tace_fail_msg("tace_tece_rotate_out_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)n_nodes), b((unsigned)((channels + 63) / 64 * 64));
#define ROT_F(TT, LL)                                                                                           \
  hipLaunchKernelGGL((k_rotout_fwd<TT, LL>), g, b, 0, s, (const TT*)m, (const TT*)alpha, (const TT*)wigner, rowptr, \
                     eid, node_map, (int)n_nodes, channels, heads, (TT*)out)
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

int tace_tece_rotate_out_bwd(int dtype, const void* m, const void* alpha, const void* wigner, const void* g_out,
                             const int32_t* rowptr, const int32_t* eid, const int32_t* node_map, int64_t n_nodes,
                             int32_t lmax, int32_t channels, int32_t heads, void* g_m, void* g_alpha, void* stream) {
  if (rotout_checks("tace_tece_rotate_out_bwd", n_nodes, lmax, channels, heads)) return -1;
  if (n_nodes == 0) return 0;
  if (!rowptr || !g_out) return tace_fail_msg("tace_tece_rotate_out_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)n_nodes), b((unsigned)((channels + 63) / 64 * 64));
#define ROT_B(TT, LL)                                                                                              \
  hipLaunchKernelGGL((k_rotout_bwd<TT, LL>), g, b, 0, s, (const TT*)m, (const TT*)alpha, (const TT*)wigner,         \
                     (const TT*)g_out, rowptr, eid, node_map, (int)n_nodes, channels, heads, (TT*)g_m, (TT*)g_alpha)
  if (dtype == TACE_F32) {
    if (lmax == 1) ROT_B(float, 1); else if (lmax == 2) ROT_B(float, 2); else ROT_B(float, 3);
  } else if (dtype == TACE_F64) {
    if (lmax == 1) ROT_B(double, 1); else if (lmax == 2) ROT_B(double, 2); else ROT_B(double, 3);
  } else {
    return tace_fail_msg("tace_tece_rotate_out_bwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef ROT_B
  return tace_check_launch("tace_tece_rotate_out_bwd");
}

}  // extern "C"
