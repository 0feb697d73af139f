// MI355X (gfx950) gate + complex edge-ACE product of the SO(2) messages
// (tace/models/_e3nn/archive/oam_2026_07_05.py:782-790) and the graph softmax
// over each receiver's in-edges (tace/models/softmax.py:100-112), forward and backward.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"
#include "tece_common.h"

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


extern "C" {

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
