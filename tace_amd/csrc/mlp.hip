// MI355X (gfx950) kernels of the radial MLP's hidden layers
// (tace/models/mlp.py:136-191: x -> silu(x W_1 a_1) -> ... -> silu(h W_L a_L),
// width 64, the last, wide layer stays a GEMM): one thread per edge keeps the
// 64 activations in registers; the (pre-scaled) weights are wave-uniform, so
// they are read through the scalar data cache into SGPRs and feed the FMAs as
// scalar operands (an LDS broadcast read would still move 64 lanes' worth of
// data per value: measured 2.6x slower forward, 1.9x backward).  The hidden
// layers then cost one pass over the radial basis in and the last hidden
// activations out instead of a GEMM + activation launch pair per layer.
//
// Layouts: radial [E, n_in]; weights packed [n_in x 64 | 64 x 64 | ...]
// (row-major, scale folded in); activations and saved pre-activations
// feature-major: h_t [64, E], z_t [n_layers, 64, E] (consecutive edges =
// consecutive addresses for every store and load).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"

int tace_fail_msg(const char* msg);   // tace_hip.hip
int tace_check_launch(const char* what);

namespace {

constexpr int W = TACE_MLP_WIDTH;

template <typename T>
__device__ __forceinline__ T sigm(T z) { return T(1) / (T(1) + exp(-z)); }

template <typename T>
__global__ __launch_bounds__(256) void k_mlp_fwd(const T* __restrict__ radial, int64_t E, int n_in, int n_layers,
                                                 const T* __restrict__ wg, T* __restrict__ h_t,
                                                 T* __restrict__ z_t) {
  const T* __restrict__ w = wg;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  T h[W], z[W];
#pragma unroll
  for (int j = 0; j < W; ++j) z[j] = T(0);
  for (int k = 0; k < n_in; ++k) {
    const T a = radial[e * n_in + k];
#pragma unroll
    for (int j = 0; j < W; ++j) z[j] += a * w[k * W + j];
  }
  int off = n_in * W;
  for (int l = 0;; ++l) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      z_t[((int64_t)l * W + j) * E + e] = z[j];
      h[j] = z[j] * sigm(z[j]);
    }
    if (l + 1 == n_layers) break;
#pragma unroll
    for (int j = 0; j < W; ++j) z[j] = T(0);
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const T a = h[k];
#pragma unroll
      for (int j = 0; j < W; ++j) z[j] += a * w[off + k * W + j];
    }
    off += W * W;
  }
#pragma unroll
  for (int j = 0; j < W; ++j) h_t[(int64_t)j * E + e] = h[j];
}

// backward to the radial basis: g_z = g_h silu'(z), g_h(prev) = W g_z
template <typename T>
__global__ __launch_bounds__(256) void k_mlp_bwd(const T* __restrict__ z_t, const T* __restrict__ gh_t, int64_t E,
                                                 int n_in, int n_layers, const T* __restrict__ wg,
                                                 T* __restrict__ g_radial) {
  const T* __restrict__ w = wg;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  T g[W];
#pragma unroll
  for (int j = 0; j < W; ++j) g[j] = gh_t[(int64_t)j * E + e];
  for (int l = n_layers - 1; l >= 0; --l) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const T zv = z_t[((int64_t)l * W + j) * E + e];
      const T s = sigm(zv);
      g[j] *= s * (T(1) + zv * (T(1) - s));
    }
    if (l == 0) break;
    const int off = n_in * W + (l - 1) * W * W;
    T gn[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      T acc = T(0);
#pragma unroll
      for (int j = 0; j < W; ++j) acc += w[off + k * W + j] * g[j];
      gn[k] = acc;
    }
#pragma unroll
    for (int k = 0; k < W; ++k) g[k] = gn[k];
  }
  for (int k = 0; k < n_in; ++k) {
    T acc = T(0);
#pragma unroll
    for (int j = 0; j < W; ++j) acc += w[k * W + j] * g[j];
    g_radial[e * n_in + k] = acc;
  }
}

int mlp_checks(const char* who, int64_t E, int32_t n_in, int32_t n_layers) {
  char msg[160];
  if (E < 0 || n_in < 1 || n_in > TACE_MLP_MAX_IN || n_layers < 1 || n_layers > TACE_MLP_MAX_LAYERS) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (n_in 1..%d, hidden layers 1..%d)", who, TACE_MLP_MAX_IN,
             TACE_MLP_MAX_LAYERS);
    return tace_fail_msg(msg);
  }
  return 0;
}

}  // namespace

extern "C" {

int tace_radial_mlp_fwd(int dtype, const void* radial, int64_t n_edges, int32_t n_in, int32_t n_layers,
                        const void* weights, void* h_t, void* z_t, void* stream) {
  if (mlp_checks("tace_radial_mlp_fwd", n_edges, n_in, n_layers)) return -1;
  if (n_edges == 0) return 0;
  if (!radial || !weights || !h_t || !z_t) return tace_fail_msg("tace_radial_mlp_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges + 255) / 256)), b(256);
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_mlp_fwd<float>, g, b, 0, s, (const float*)radial, n_edges, n_in, n_layers,
                       (const float*)weights, (float*)h_t, (float*)z_t);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_mlp_fwd<double>, g, b, 0, s, (const double*)radial, n_edges, n_in, n_layers,
                       (const double*)weights, (double*)h_t, (double*)z_t);
  else
    return tace_fail_msg("tace_radial_mlp_fwd: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_radial_mlp_fwd");
}

int tace_radial_mlp_bwd(int dtype, const void* z_t, const void* g_h_t, int64_t n_edges, int32_t n_in,
                        int32_t n_layers, const void* weights, void* g_radial, void* stream) {
  if (mlp_checks("tace_radial_mlp_bwd", n_edges, n_in, n_layers)) return -1;
  if (n_edges == 0) return 0;
  if (!z_t || !g_h_t || !weights || !g_radial) return tace_fail_msg("tace_radial_mlp_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges + 255) / 256)), b(256);
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_mlp_bwd<float>, g, b, 0, s, (const float*)z_t, (const float*)g_h_t, n_edges, n_in,
                       n_layers, (const float*)weights, (float*)g_radial);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_mlp_bwd<double>, g, b, 0, s, (const double*)z_t, (const double*)g_h_t, n_edges,
                       n_in, n_layers, (const double*)weights, (double*)g_radial);
  else
    return tace_fail_msg("tace_radial_mlp_bwd: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_radial_mlp_bwd");
}

}  // extern "C"
