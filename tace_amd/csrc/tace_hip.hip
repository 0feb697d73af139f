// MI355X (gfx950) kernels of the TACE energy/force path, exported through a
// flat C ABI (include/tace_hip.h).  Host code (tace_amd/*.py) owns every
// buffer; the library never allocates and never synchronises the stream.
//
// Contents
//   * edge featurisation: Bessel j0 x C2-polynomial cutoff radial basis and
//     component-normalised real spherical harmonics, forward and the backward
//     to edge vectors (tace/models/radial.py:43-84, 437-472, 974-993;
//     tace/models/angular.py:288-315);
//   * CG tensor products: generated kernels (gen/tp_kernels.inc) dispatched by
//     variant key (tace/models/_e3nn/fused.py:17-95, 172-271);
//   * periodic cell-list neighbour search, float64, same edge set as
//     tace/dataset/neighbour_list.py:195-298 (matscipy "ijSd").
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/tace_hip.h"

namespace {

thread_local char g_err[512] = "";
// tace_mark_phase_event: recorded after the next edge-TP backward's product
// kernel on this host thread, then cleared
thread_local hipEvent_t g_phase_event = nullptr;

int fail(const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return -1;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
    return -2;
  }
  return 0;
}

}  // namespace

extern "C" int tace_mark_phase_event(void* hip_event) {
  g_phase_event = (hipEvent_t)hip_event;
  return 0;
}

// error helpers shared with the other translation units of the library
int tace_fail_msg(const char* msg) { return fail(msg); }
int tace_check_launch(const char* what) { return check_launch(what); }

#include "common.h"
#include "gen/registry.inc"
#include "gen/sh.inc"

// ---------------------------------------------------------------- helpers --
template <typename T>
__global__ void k_fill(T* p, size_t n, T v) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

template <typename T>
static void launch_fill(T* p, size_t n, T v, hipStream_t s) {
  if (n == 0) return;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_fill<T>, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
}

// gx[s, :] = sum over the receiver-sorted slots k listed for sender s of
// cbuf[k, :]; fixed summation order (sender CSR), no atomics.  A cbuf row has
// `row` values; with sg.n > 0 it is split into segments (offset, length) and
// segment g of sender s goes to gx[n * off_g + s * len_g ...] (the
// group-major batch layout), else the row goes to gx[s * row ...].
// V values per thread (vector loads); row, offsets and lengths are multiples of V.
struct RowSegs {
  int n;
  int64_t off[8], len[8];
};

template <typename T, int V>
__global__ __launch_bounds__(256) void k_seg_rowsum(const T* __restrict__ cbuf, const int* __restrict__ s_rowptr,
                                                    const int* __restrict__ s_slot, const int* __restrict__ map,
                                                    T* __restrict__ gx, int n, int64_t row, RowSegs sg) {
  typedef T vec __attribute__((ext_vector_type(V)));
  const int s0 = blockIdx.x;
  if (s0 >= n) return;
  const int b = s_rowptr[s0], e = s_rowptr[s0 + 1];
  const int s = map ? map[s0] : s0;  // feature row of the sender
  for (int64_t j = (int64_t)threadIdx.x * V; j < row; j += 256 * V) {
    vec acc = (vec)(T(0));
#pragma unroll 4
    for (int k = b; k < e; ++k) acc += __builtin_nontemporal_load((const vec*)(cbuf + (size_t)s_slot[k] * row + j));
    int64_t dst = (int64_t)s * row + j;
    for (int g = 0; g < sg.n; ++g)
      if (j >= sg.off[g] && j < sg.off[g] + sg.len[g]) dst = (int64_t)n * sg.off[g] + (int64_t)s * sg.len[g] + (j - sg.off[g]);
    *(vec*)(gx + dst) = acc;
  }
}

template <typename T>
static void launch_seg_rowsum(const T* cbuf, const int* s_rowptr, const int* s_slot, const int* map, T* gx, int n,
                              int64_t row, const RowSegs& sg, int C, hipStream_t st) {
  const int v = 16 / (int)sizeof(T);
  if (C % v == 0)
    hipLaunchKernelGGL((k_seg_rowsum<T, 16 / sizeof(T)>), dim3((unsigned)n), dim3(256), 0, st, cbuf, s_rowptr, s_slot,
                       map, gx, n, row, sg);
  else
    hipLaunchKernelGGL((k_seg_rowsum<T, 1>), dim3((unsigned)n), dim3(256), 0, st, cbuf, s_rowptr, s_slot, map, gx, n,
                       row, sg);
}

// out[target[s], :] += sum over k in [rowptr[s], rowptr[s+1]) of
// rows[slot ? slot[k] : k, :] -- a segmented row sum in fixed (slot) order,
// added into out; target = null means target[s] = s.  One workgroup per
// segment; V values per thread (vector loads).  A target row must not occur
// in two segments of one launch.
template <typename T, int V>
__global__ __launch_bounds__(256) void k_rows_accumulate(const T* __restrict__ rows, int64_t width,
                                                         const int* __restrict__ rowptr, const int* __restrict__ slot,
                                                         const int* __restrict__ target, int n_seg,
                                                         T* __restrict__ out, int run) {
  typedef T vec __attribute__((ext_vector_type(V)));
  const int sg = blockIdx.x;
  if (sg >= n_seg) return;
  const int b = rowptr[sg], e = rowptr[sg + 1];
  if (b == e) return;
  const int64_t t = target ? (int64_t)target[sg] : (int64_t)sg;
  for (int64_t j = (int64_t)threadIdx.x * V; j < width; j += 256 * V) {
    vec acc = (vec)(T(0));
    // run > 1: only the segment's first position and the multiples of run
    // inside it hold rows (the other positions are parts of those runs)
    for (int k = b; k < e; k = run > 1 ? (k / run + 1) * run : k + 1) {
      const int64_t r = slot ? (int64_t)slot[k] : (int64_t)k;
      acc += __builtin_nontemporal_load((const vec*)(rows + r * width + j));
    }
    vec* o = (vec*)(out + t * width + j);
    *o = *o + acc;
  }
}

// out[g, j] = sum of v[k, j] over the rows k in [ptr[g], ptr[g+1]): one
// workgroup per graph, thread t sums rows ptr[g] + t + 256 i in order, then a
// fixed tree over the 256 partial sums -- the same bits on every run.
template <typename T>
__global__ __launch_bounds__(256) void k_graph_sum(const T* __restrict__ v, int64_t width,
                                                   const int64_t* __restrict__ ptr, T* __restrict__ out) {
  __shared__ T sh[256];
  const int g = (int)blockIdx.x, t = (int)threadIdx.x;
  const int64_t b = ptr[g], e = ptr[g + 1];
  for (int64_t j = 0; j < width; ++j) {
    T acc = T(0);
    for (int64_t k = b + t; k < e; k += 256) acc += v[k * width + j];
    sh[t] = acc;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (t < o) sh[t] += sh[t + o];
      __syncthreads();
    }
    if (t == 0) out[(int64_t)g * width + j] = sh[0];
    __syncthreads();
  }
}

// out[r, j] = bias[j] + sum_i x[r, i] m[i, j] for narrow matrices (k, n <= 64):
// one thread per output element; the row's k inputs come from L1 / L2 (n
// threads share a row), m and bias are a few hundred bytes that stay in L1
template <typename T>
__global__ __launch_bounds__(256) void k_narrow_linear(const T* __restrict__ x, int64_t n_rows, int k,
                                                       const T* __restrict__ m, const T* __restrict__ bias, int n,
                                                       T* __restrict__ out) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= n_rows * n) return;
  const int64_t r = id / n;
  const int j = (int)(id - r * n);
  T acc = bias ? bias[j] : T(0);
  const T* xr = x + r * k;
  for (int i = 0; i < k; ++i) acc += xr[i] * m[(int64_t)i * n + j];
  out[id] = acc;
}

// gy = sum of the per-part grad_y partials, in part order (added to what out
// holds when accumulate != 0)
template <typename T>
__global__ __launch_bounds__(256) void k_sum_parts(const T* __restrict__ parts, int nparts, int64_t n,
                                                   T* __restrict__ out, int accumulate = 0) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  T acc = parts[i];
  for (int q = 1; q < nparts; ++q) acc += parts[(size_t)q * n + i];
  out[i] = accumulate ? out[i] + acc : acc;
}

// the same, four float32 per thread (n % 4 == 0, 16-byte aligned arrays):
// the same sums in the same order, a quarter of the memory instructions
typedef float sp_f4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_sum_parts4(const float* __restrict__ parts, int nparts, int64_t n,
                                                    float* __restrict__ out, int accumulate) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  sp_f4 acc = *(const sp_f4*)(parts + i);
  for (int q = 1; q < nparts; ++q) acc += *(const sp_f4*)(parts + (size_t)q * n + i);
  if (accumulate) acc = *(const sp_f4*)(out + i) + acc;
  *(sp_f4*)(out + i) = acc;
}

// k_sum_parts for float32, on four elements per thread where the sizes and
// alignment allow
static void sum_parts_f32(const float* parts, int nparts, int64_t n, float* out, int accumulate, hipStream_t s) {
  if (n <= 0) return;
  if ((n & 3) == 0 && ((((uintptr_t)parts) | ((uintptr_t)out)) & 15) == 0) {
    hipLaunchKernelGGL(k_sum_parts4, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, parts, nparts, n, out,
                       accumulate);
  } else {
    hipLaunchKernelGGL(k_sum_parts<float>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, parts, nparts, n,
                       out, accumulate);
  }
}

// ------------------------------------------------------------ edge vectors --
// vec[e] = pos[dst] - pos[src] + S[e] . lat[eb[e]]   (adapter.py:334-340)
template <typename T>
__global__ __launch_bounds__(256) void k_edge_vec_fwd(const T* __restrict__ pos, const T* __restrict__ lat,
                                                      const int* __restrict__ src, const int* __restrict__ dst,
                                                      const T* __restrict__ shift, const int* __restrict__ eb,
                                                      int64_t E, T* __restrict__ vec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int i = src[e], j = dst[e];
  const T* L = lat + (size_t)(eb ? eb[e] : 0) * 9;
  const T s0 = shift[3 * e], s1 = shift[3 * e + 1], s2 = shift[3 * e + 2];
#pragma unroll
  for (int c = 0; c < 3; ++c)
    vec[3 * e + c] = pos[3 * j + c] - pos[3 * i + c] + (s0 * L[c] + s1 * L[3 + c] + s2 * L[6 + c]);
}

// gpos[n] = sum_{e: dst(e)=n} g[e] - sum_{e: src(e)=n} g[e], both in CSR order
template <typename T>
__global__ __launch_bounds__(256) void k_edge_vec_bwd(const T* __restrict__ g, const int* __restrict__ rowptr,
                                                      const int* __restrict__ eid, const int* __restrict__ s_rowptr,
                                                      const int* __restrict__ s_slot, int n, T* __restrict__ gpos) {
  const int a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= n) return;
  T x = T(0), y = T(0), z = T(0);
  for (int k = rowptr[a]; k < rowptr[a + 1]; ++k) {
    const int e = eid ? eid[k] : k;
    x += g[3 * e];
    y += g[3 * e + 1];
    z += g[3 * e + 2];
  }
  for (int k = s_rowptr[a]; k < s_rowptr[a + 1]; ++k) {
    const int sl = s_slot[k];
    const int e = eid ? eid[sl] : sl;
    x -= g[3 * e];
    y -= g[3 * e + 1];
    z -= g[3 * e + 2];
  }
  gpos[3 * a] = x;
  gpos[3 * a + 1] = y;
  gpos[3 * a + 2] = z;
}

// ------------------------------------------------------ edge featurisation --
// R[e, n] = pref * sin(b_n r) / r * f(r / rc) * [r < rc],  r = |v| + 1e-9
// f(x) = 1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2)
// Y[e, :] = SH_lmax(v / r)
template <typename T>
__device__ __forceinline__ T ipow(T x, int p) {
  T r = T(1);
  for (int i = 0; i < p; ++i) r *= x;
  return r;
}

template <typename T, int LMAX>
__global__ __launch_bounds__(256) void k_edge_basis_fwd(const T* __restrict__ vec, int64_t E, int nb,
                                                        const T* __restrict__ bw, T pref, T rc, int p,
                                                        T* __restrict__ R, T* __restrict__ Y) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const T vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
  const T nrm = sqrt(vx * vx + vy * vy + vz * vz);
  const T r = nrm + T(1e-9);
  const T x = r / rc;
  const T c1 = T((p + 1.0) * (p + 2.0) / 2.0), c2 = T(p * (p + 2.0)), c3 = T(p * (p + 1.0) / 2.0);
  const T xp = ipow(x, p);
  T env = T(1) - c1 * xp + c2 * (xp * x) - c3 * (xp * x * x);
  env = (r < rc) ? env : T(0);
  for (int n = 0; n < nb; ++n) R[e * nb + n] = pref * (sin(bw[n] * r) / r) * env;
  constexpr int DY = (LMAX + 1) * (LMAX + 1);
  T o[DY];
  const T ux = vx / r, uy = vy / r, uz = vz / r;
  if constexpr (LMAX == 0) sh_eval_0<T>(ux, uy, uz, o);
  if constexpr (LMAX == 1) sh_eval_1<T>(ux, uy, uz, o);
  if constexpr (LMAX == 2) sh_eval_2<T>(ux, uy, uz, o);
  if constexpr (LMAX == 3) sh_eval_3<T>(ux, uy, uz, o);
#pragma unroll
  for (int i = 0; i < DY; ++i) Y[e * DY + i] = o[i];
}

template <typename T, int LMAX>
__global__ __launch_bounds__(256) void k_edge_basis_bwd(const T* __restrict__ vec, const T* __restrict__ gR,
                                                        const T* __restrict__ gY, int64_t E, int nb,
                                                        const T* __restrict__ bw, T pref, T rc, int p,
                                                        T* __restrict__ gvec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const T vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
  const T nrm = sqrt(vx * vx + vy * vy + vz * vz);
  const T r = nrm + T(1e-9);
  const T x = r / rc;
  const T c1 = T((p + 1.0) * (p + 2.0) / 2.0), c2 = T(p * (p + 2.0)), c3 = T(p * (p + 1.0) / 2.0);
  const T xp = ipow(x, p);
  const T xpm1 = ipow(x, p - 1);
  T env = T(1) - c1 * xp + c2 * (xp * x) - c3 * (xp * x * x);
  T denv = (-c1 * T(p) * xpm1 + c2 * T(p + 1) * xp - c3 * T(p + 2) * (xp * x)) / rc;
  const bool in = r < rc;
  env = in ? env : T(0);
  denv = in ? denv : T(0);
  T gr = T(0);
  for (int n = 0; n < nb; ++n) {
    const T b = bw[n];
    const T sn = sin(b * r), cs = cos(b * r);
    const T dRdr = pref * (((b * cs) * r - sn) / (r * r) * env + (sn / r) * denv);
    gr += gR[e * nb + n] * dRdr;
  }
  constexpr int DY = (LMAX + 1) * (LMAX + 1);
  const T ux = vx / r, uy = vy / r, uz = vz / r;
  T gux = T(0), guy = T(0), guz = T(0);
  if constexpr (LMAX == 0) sh_grad_0<T>(ux, uy, uz, gY + e * DY, gux, guy, guz);
  if constexpr (LMAX == 1) sh_grad_1<T>(ux, uy, uz, gY + e * DY, gux, guy, guz);
  if constexpr (LMAX == 2) sh_grad_2<T>(ux, uy, uz, gY + e * DY, gux, guy, guz);
  if constexpr (LMAX == 3) sh_grad_3<T>(ux, uy, uz, gY + e * DY, gux, guy, guz);
  // u = v / r, r = |v| + eps:  du_a/dv_b = d_ab / r - v_a v_b / (|v| r^2)
  const T gdot = gux * vx + guy * vy + guz * vz;
  const T k = gdot / (nrm * r * r);
  const T gl = gr / nrm;
  gvec[3 * e] = gux / r - vx * k + gl * vx;
  gvec[3 * e + 1] = guy / r - vy * k + gl * vy;
  gvec[3 * e + 2] = guz / r - vz * k + gl * vz;
}

template <typename T>
static int edge_basis_fwd_t(const T* vec, int64_t E, int nb, const T* bw, double pref, double rc, int p, int lmax,
                            T* R, T* Y, hipStream_t s) {
  if (E <= 0) return 0;
  dim3 g((unsigned)((E + 255) / 256)), b(256);
  switch (lmax) {
    case 0: hipLaunchKernelGGL((k_edge_basis_fwd<T, 0>), g, b, 0, s, vec, E, nb, bw, (T)pref, (T)rc, p, R, Y); break;
    case 1: hipLaunchKernelGGL((k_edge_basis_fwd<T, 1>), g, b, 0, s, vec, E, nb, bw, (T)pref, (T)rc, p, R, Y); break;
    case 2: hipLaunchKernelGGL((k_edge_basis_fwd<T, 2>), g, b, 0, s, vec, E, nb, bw, (T)pref, (T)rc, p, R, Y); break;
    case 3: hipLaunchKernelGGL((k_edge_basis_fwd<T, 3>), g, b, 0, s, vec, E, nb, bw, (T)pref, (T)rc, p, R, Y); break;
    default: return fail("tace_edge_basis_fwd: lmax must be 0..3");
  }
  return check_launch("tace_edge_basis_fwd");
}

template <typename T>
static int edge_basis_bwd_t(const T* vec, const T* gR, const T* gY, int64_t E, int nb, const T* bw, double pref,
                            double rc, int p, int lmax, T* gvec, hipStream_t s) {
  if (E <= 0) return 0;
  dim3 g((unsigned)((E + 255) / 256)), b(256);
  switch (lmax) {
    case 0: hipLaunchKernelGGL((k_edge_basis_bwd<T, 0>), g, b, 0, s, vec, gR, gY, E, nb, bw, (T)pref, (T)rc, p, gvec); break;
    case 1: hipLaunchKernelGGL((k_edge_basis_bwd<T, 1>), g, b, 0, s, vec, gR, gY, E, nb, bw, (T)pref, (T)rc, p, gvec); break;
    case 2: hipLaunchKernelGGL((k_edge_basis_bwd<T, 2>), g, b, 0, s, vec, gR, gY, E, nb, bw, (T)pref, (T)rc, p, gvec); break;
    case 3: hipLaunchKernelGGL((k_edge_basis_bwd<T, 3>), g, b, 0, s, vec, gR, gY, E, nb, bw, (T)pref, (T)rc, p, gvec); break;
    default: return fail("tace_edge_basis_bwd: lmax must be 0..3");
  }
  return check_launch("tace_edge_basis_bwd");
}

// ------------------------------------------------------------ neighbours --
struct NlGeom {
  double cell[9];  // rows are lattice vectors
  double inv[9];   // inverse of cell (frac = pos @ inv)
  int pbc[3];
  int nb[3];       // bins per axis
  int reach[3];    // bins searched on each side
  double rc2;
};

static void inv3(const double* a, double* o) {
  double det = a[0] * (a[4] * a[8] - a[5] * a[7]) - a[1] * (a[3] * a[8] - a[5] * a[6]) +
               a[2] * (a[3] * a[7] - a[4] * a[6]);
  o[0] = (a[4] * a[8] - a[5] * a[7]) / det;
  o[1] = (a[2] * a[7] - a[1] * a[8]) / det;
  o[2] = (a[1] * a[5] - a[2] * a[4]) / det;
  o[3] = (a[5] * a[6] - a[3] * a[8]) / det;
  o[4] = (a[0] * a[8] - a[2] * a[6]) / det;
  o[5] = (a[2] * a[3] - a[0] * a[5]) / det;
  o[6] = (a[3] * a[7] - a[4] * a[6]) / det;
  o[7] = (a[1] * a[6] - a[0] * a[7]) / det;
  o[8] = (a[0] * a[4] - a[1] * a[3]) / det;
}

static int nl_geometry(const double* cell, const int32_t* pbc, double cutoff, NlGeom* g) {
  if (!(cutoff > 0.0)) return fail("tace_nl: cutoff must be > 0");
  memcpy(g->cell, cell, 9 * sizeof(double));
  double det = cell[0] * (cell[4] * cell[8] - cell[5] * cell[7]) - cell[1] * (cell[3] * cell[8] - cell[5] * cell[6]) +
               cell[2] * (cell[3] * cell[7] - cell[4] * cell[6]);
  if (fabs(det) < 1e-12) return fail("tace_nl: cell is singular (complete the cell for non-periodic axes)");
  inv3(cell, g->inv);
  for (int k = 0; k < 3; ++k) {
    g->pbc[k] = pbc[k] ? 1 : 0;
    const double c0 = g->inv[k], c1 = g->inv[3 + k], c2 = g->inv[6 + k];
    const double h = 1.0 / sqrt(c0 * c0 + c1 * c1 + c2 * c2);  // plane spacing
    int nb = (int)floor(h / cutoff);
    if (nb < 1) nb = 1;
    if (nb > 512) nb = 512;
    g->nb[k] = nb;
    g->reach[k] = (int)ceil(cutoff * nb / h + 1e-9);
    if (!g->pbc[k] && g->reach[k] > nb) g->reach[k] = nb;
  }
  g->rc2 = cutoff * cutoff;
  return 0;
}

__global__ void k_nl_bin(const double* __restrict__ pos, int n, NlGeom g, int* __restrict__ abin,
                         int* __restrict__ aimg, int* __restrict__ bcount) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double px = pos[3 * i], py = pos[3 * i + 1], pz = pos[3 * i + 2];
  int b[3];
  for (int k = 0; k < 3; ++k) {
    const double f = px * g.inv[k] + py * g.inv[3 + k] + pz * g.inv[6 + k];
    int o = 0;
    double w = f;
    if (g.pbc[k]) {
      o = (int)floor(f);
      w = f - (double)o;
    }
    int bi = (int)floor(w * g.nb[k]);
    bi = bi < 0 ? 0 : (bi >= g.nb[k] ? g.nb[k] - 1 : bi);
    b[k] = bi;
    aimg[3 * i + k] = o;
  }
  const int lin = (b[0] * g.nb[1] + b[1]) * g.nb[2] + b[2];
  abin[i] = lin;
  atomicAdd(bcount + lin, 1);
}

// ---- edge pairs: the two directions of an edge ---------------------------
// partner[e] = id of the reverse of edge e (sender i -> receiver j, shift S):
// the edge j -> i with shift -S, looked up among receiver i's edges; -1 when
// the list has none.  One wavefront per receiver j walks its edges; for each,
// the 64 lanes test 64 of receiver i's edges at a time (coalesced reads) and
// a ballot picks the match.
__global__ __launch_bounds__(64) void k_edge_partner(const int* __restrict__ rowptr, const int* __restrict__ eid,
                                                     const int* __restrict__ src, const int* __restrict__ shifts,
                                                     int* __restrict__ partner) {
  const int j = (int)blockIdx.x, lane = (int)threadIdx.x;
  const int end = rowptr[j + 1];
  for (int k = rowptr[j]; k < end; ++k) {
    const int e = eid ? eid[k] : k;
    const int i = src[e];
    const int sx = -shifts[3 * e], sy = -shifts[3 * e + 1], sz = -shifts[3 * e + 2];
    int found = -1;
    const int b2 = rowptr[i], e2end = rowptr[i + 1];
    for (int k2 = b2; k2 < e2end && found < 0; k2 += 64) {
      const int kk = k2 + lane;
      bool hit = false;
      int e2 = 0;
      if (kk < e2end) {
        e2 = eid ? eid[kk] : kk;
        hit = src[e2] == j && shifts[3 * e2] == sx && shifts[3 * e2 + 1] == sy && shifts[3 * e2 + 2] == sz;
      }
      const unsigned long long m = __ballot(hit);
      if (m) found = __shfl(e2, __ffsll((long long)m) - 1);
    }
    if (lane == 0) partner[e] = found;
  }
}

// Exclusive scan of m ints in three launches (1024 elements per block):
// block sums, a scan of the sums (k_scan), then each block's own scan plus
// its offset.  out[m] = total.
__device__ __forceinline__ int block_excl_scan256(int v, int* sh) {
  const int t = (int)threadIdx.x;
  sh[t] = v;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {
    const int u = t >= o ? sh[t - o] : 0;
    __syncthreads();
    sh[t] += u;
    __syncthreads();
  }
  const int incl = sh[t];
  __syncthreads();
  return incl - v;
}

__global__ __launch_bounds__(256) void k_scan_sums(const int* __restrict__ cnt, int m, int* __restrict__ sums) {
  __shared__ int sh[256];
  const int base = (int)blockIdx.x * 1024 + 4 * (int)threadIdx.x;
  int v = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) v += base + q < m ? cnt[base + q] : 0;
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) sh[threadIdx.x] += sh[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) sums[blockIdx.x] = sh[0];
}

__global__ __launch_bounds__(256) void k_scan_apply(const int* __restrict__ cnt, int m,
                                                    const int* __restrict__ offs, int* __restrict__ out) {
  __shared__ int sh[256];
  const int base = (int)blockIdx.x * 1024 + 4 * (int)threadIdx.x;
  int v[4], tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[q] = base + q < m ? cnt[base + q] : 0;
    tot += v[q];
  }
  int run = offs[blockIdx.x] + block_excl_scan256(tot, sh);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (base + q < m) out[base + q] = run;
    run += v[q];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 255) out[m] = run;
}

// The partner of e when the pairing is mutual, else -1: a zero-shift self
// edge finds itself, and of duplicated edges only the first pair is mutual;
// every other copy keeps a row of its own.
__device__ __forceinline__ int mutual_partner(const int* __restrict__ partner, int e) {
  const int p = partner[e];
  return (p >= 0 && p != e && partner[p] == e) ? p : -1;
}

// owner[e] = 1 when e carries its pair's row (the lower id of a pair, or an
// edge without a partner)
__global__ void k_edge_owner(const int* __restrict__ partner, int E, int* __restrict__ owner) {
  const int e = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (e >= E) return;
  const int p = mutual_partner(partner, e);
  owner[e] = (p < 0 || p > e) ? 1 : 0;
}

// rank = exclusive scan of owner: w_rows[e] = the row of e's pair;
// row_edges[r] / row_partner[r] = the owner edge of row r and its partner
__global__ void k_edge_rows(const int* __restrict__ partner, const int* __restrict__ rank, int E,
                            int* __restrict__ w_rows, int* __restrict__ row_edges, int* __restrict__ row_partner) {
  const int e = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (e >= E) return;
  const int p = mutual_partner(partner, e);
  if (p < 0 || p > e) {
    const int r = rank[e];
    w_rows[e] = r;
    row_edges[r] = e;
    row_partner[r] = p;
  } else {
    w_rows[e] = rank[p];
  }
}

// exclusive scan of cnt[0..m) into out[0..m]; single block of 1024 threads
__global__ __launch_bounds__(1024) void k_scan(const int* __restrict__ cnt, int m, int* __restrict__ out) {
  __shared__ long long part[1024];
  const int t = threadIdx.x;
  const int chunk = (m + 1023) / 1024;
  const int b = t * chunk, e = min(m, b + chunk);
  long long s = 0;
  for (int i = b; i < e; ++i) s += cnt[i];
  part[t] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    long long v = (t >= o) ? part[t - o] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  long long run = part[t] - s;
  for (int i = b; i < e; ++i) {
    out[i] = (int)run;
    run += cnt[i];
  }
  if (t == 1023) out[m] = (int)part[1023];
}

__global__ void k_nl_scatter(const int* __restrict__ abin, int n, const int* __restrict__ bstart,
                             int* __restrict__ bfill, int* __restrict__ batoms) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int b = abin[i];
  const int slot = atomicAdd(bfill + b, 1);
  batoms[bstart[b] + slot] = i;
}

// ------------------------------------------------- batched neighbours --
// Many structures in one pass.  The host-built plan table holds per structure
// its NlGeom, then struct_ptr[ns+1] (first atom of each structure) and
// bin_off[ns+1] (first bin of each structure in the batch's bin arrays).
// Atoms, bins and batoms entries are batch-global ids; the search per
// receiver is the single-structure one (same candidate order, same distance
// arithmetic), so each structure's edges come out exactly as
// tace_nl_count/_fill produce them.
struct NlBatch {
  const NlGeom* geo;
  const int* sptr;
  const int* boff;
  int ns;
};

static __device__ __forceinline__ int nlb_struct_of(const NlBatch& B, int a) {
  int lo = 0, hi = B.ns - 1;   // last s with sptr[s] <= a
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (B.sptr[mid] <= a) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ void k_nlb_bin(const double* __restrict__ pos, int n, NlBatch B, int* __restrict__ abin,
                          int* __restrict__ aimg, int* __restrict__ bcount) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int s = nlb_struct_of(B, i);
  const NlGeom& g = B.geo[s];
  const double px = pos[3 * i], py = pos[3 * i + 1], pz = pos[3 * i + 2];
  int b[3];
  for (int k = 0; k < 3; ++k) {
    const double f = px * g.inv[k] + py * g.inv[3 + k] + pz * g.inv[6 + k];
    int o = 0;
    double w = f;
    if (g.pbc[k]) {
      o = (int)floor(f);
      w = f - (double)o;
    }
    int bi = (int)floor(w * g.nb[k]);
    bi = bi < 0 ? 0 : (bi >= g.nb[k] ? g.nb[k] - 1 : bi);
    b[k] = bi;
    aimg[3 * i + k] = o;
  }
  const int lin = B.boff[s] + (b[0] * g.nb[1] + b[1]) * g.nb[2] + b[2];
  abin[i] = lin;
  atomicAdd(bcount + lin, 1);
}

// Deterministic bin contents without a sort: atom i goes to the slot of its
// rank (by id) among the atoms k_nl_scatter put into its bin in arbitrary
// order -- batoms ends up ascending in every bin, with a thread per atom
// instead of a serial sort per bin (single structures and batches alike).
__global__ void k_nlb_rank(const int* __restrict__ abin, int n, const int* __restrict__ bstart,
                           const int* __restrict__ unsorted, int* __restrict__ batoms) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int b = abin[i];
  const int q0 = bstart[b], q1 = bstart[b + 1];
  int r = 0;
  for (int q = q0; q < q1; ++q) r += unsorted[q] < i;
  batoms[q0 + r] = i;
}

// is source b (with periodic shift S) within the cutoff of receiver a?  The
// brute-force oracle's arithmetic (no contraction), the self image excluded.
static __device__ __forceinline__ bool nl_pair(const double* __restrict__ pos, const int* __restrict__ aimg,
                                               const NlGeom& g, int a, double ax, double ay, double az,
                                               const int* oa, int sx, int sy, int sz, int b, int* S) {
#pragma clang fp contract(off)
  S[0] = aimg[3 * b] - oa[0] - sx;
  S[1] = aimg[3 * b + 1] - oa[1] - sy;
  S[2] = aimg[3 * b + 2] - oa[2] - sz;
  if (b == a && S[0] == 0 && S[1] == 0 && S[2] == 0) return false;
  const double d0 = ax - pos[3 * b], d1 = ay - pos[3 * b + 1], d2 = az - pos[3 * b + 2];
  const double s0 = (double)S[0], s1 = (double)S[1], s2 = (double)S[2];
  const double v0 = d0 + s0 * g.cell[0] + s1 * g.cell[3] + s2 * g.cell[6];
  const double v1 = d1 + s0 * g.cell[1] + s1 * g.cell[4] + s2 * g.cell[7];
  const double v2 = d2 + s0 * g.cell[2] + s1 * g.cell[5] + s2 * g.cell[8];
  const double r2 = v0 * v0 + v1 * v1 + v2 * v2;
  return r2 < g.rc2;
}

// For receiver a: every source b and shift S with |r_a - r_b + S.cell|^2 < rc^2,
// (b, S) != (a, 0) (nl_pair: the distance exactly as the brute-force oracle
// evaluates it for edge (i=b, j=a, S)).  WAVE = false: one thread per receiver;
// WAVE = true: one wavefront per receiver (four per workgroup), the 64 lanes
// over each bin's candidates, counts by ballot and fill slots by the rank of
// the lane's hit among the wave's hits, so the edge order is the serial one.
// A structure of n atoms gives only n / 64 wavefronts with a thread per
// receiver; below NL_WAVE_MAX atoms the wavefront form fills the GPU.
constexpr int NL_WAVE_MAX = 32768;

template <bool FILL, bool WAVE>
__global__ __launch_bounds__(256) void k_nl_edges(const double* __restrict__ pos, int n, NlGeom g,
                                                  const int* __restrict__ abin, const int* __restrict__ aimg,
                                                  const int* __restrict__ bstart, const int* __restrict__ batoms,
                                                  int* __restrict__ counts, const int* __restrict__ rowptr,
                                                  int* __restrict__ src, int* __restrict__ shift) {
  const int lane = WAVE ? (int)(threadIdx.x & 63) : 0;
  const int a = WAVE ? (int)(blockIdx.x * 4 + (threadIdx.x >> 6)) : (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (a >= n) return;
  const double ax = pos[3 * a], ay = pos[3 * a + 1], az = pos[3 * a + 2];
  const int lin = abin[a];
  const int ba[3] = {lin / (g.nb[1] * g.nb[2]), (lin / g.nb[2]) % g.nb[1], lin % g.nb[2]};
  const int oa[3] = {aimg[3 * a], aimg[3 * a + 1], aimg[3 * a + 2]};
  int cnt = 0;
  const int base = FILL ? rowptr[a] : 0;
  int lo[3], hi[3];
  for (int k = 0; k < 3; ++k) {
    lo[k] = ba[k] - g.reach[k];
    hi[k] = ba[k] + g.reach[k];
    if (!g.pbc[k]) {
      lo[k] = lo[k] < 0 ? 0 : lo[k];
      hi[k] = hi[k] >= g.nb[k] ? g.nb[k] - 1 : hi[k];
    }
  }
  for (int bx = lo[0]; bx <= hi[0]; ++bx) {
    const int wx = ((bx % g.nb[0]) + g.nb[0]) % g.nb[0];
    const int sx = (bx - wx) / g.nb[0];
    for (int by = lo[1]; by <= hi[1]; ++by) {
      const int wy = ((by % g.nb[1]) + g.nb[1]) % g.nb[1];
      const int sy = (by - wy) / g.nb[1];
      for (int bz = lo[2]; bz <= hi[2]; ++bz) {
        const int wz = ((bz % g.nb[2]) + g.nb[2]) % g.nb[2];
        const int sz = (bz - wz) / g.nb[2];
        const int bl = (wx * g.nb[1] + wy) * g.nb[2] + wz;
        const int q1 = bstart[bl + 1];
        for (int q0 = bstart[bl]; q0 < q1; q0 += (WAVE ? 64 : 1)) {
          const int q = q0 + lane;
          int S[3] = {0, 0, 0};
          int b = 0;
          bool hit = false;
          if (q < q1) {
            b = batoms[q];
            hit = nl_pair(pos, aimg, g, a, ax, ay, az, oa, sx, sy, sz, b, S);
          }
          if (WAVE) {
            const unsigned long long m = __ballot(hit);
            if (FILL && hit) {
              const int slot = base + cnt + __popcll(m & ((1ull << lane) - 1ull));
              src[slot] = b;
              shift[3 * slot] = S[0];
              shift[3 * slot + 1] = S[1];
              shift[3 * slot + 2] = S[2];
            }
            cnt += __popcll(m);
          } else if (hit) {
            if (FILL) {
              const int slot = base + cnt;
              src[slot] = b;
              shift[3 * slot] = S[0];
              shift[3 * slot + 1] = S[1];
              shift[3 * slot + 2] = S[2];
            }
            ++cnt;
          }
        }
      }
    }
  }
  if (!FILL && lane == 0) counts[a] = cnt;
}

// WAVE = false: one thread per receiver (large structures: enough receivers
// to fill the GPU).  WAVE = true: one wavefront per receiver, the 64 lanes
// over each bin's candidates; counts by ballot, fill slots by the rank of the
// lane's hit among the wave's hits -- the candidate order, and so the edge
// order, is the serial one (small structures, where a thread per receiver
// would leave the GPU idle behind a few long serial loops).
template <bool FILL, bool WAVE>
__global__ __launch_bounds__(256) void k_nlb_edges(const double* __restrict__ pos, int n, NlBatch B,
                                                   const int* __restrict__ abin, const int* __restrict__ aimg,
                                                   const int* __restrict__ bstart, const int* __restrict__ batoms,
                                                   int* __restrict__ counts, const int* __restrict__ rowptr,
                                                   int* __restrict__ src, int* __restrict__ shift) {
  const int lane = WAVE ? (int)(threadIdx.x & 63) : 0;
  const int a = WAVE ? (int)(blockIdx.x * 4 + (threadIdx.x >> 6)) : (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (a >= n) return;
  const int s = nlb_struct_of(B, a);
  const NlGeom& g = B.geo[s];
  const int b0 = B.boff[s];
  const double ax = pos[3 * a], ay = pos[3 * a + 1], az = pos[3 * a + 2];
  const int lin = abin[a] - b0;
  const int ba[3] = {lin / (g.nb[1] * g.nb[2]), (lin / g.nb[2]) % g.nb[1], lin % g.nb[2]};
  const int oa[3] = {aimg[3 * a], aimg[3 * a + 1], aimg[3 * a + 2]};
  int cnt = 0;
  const int base = FILL ? rowptr[a] : 0;
  int lo[3], hi[3];
  for (int k = 0; k < 3; ++k) {
    lo[k] = ba[k] - g.reach[k];
    hi[k] = ba[k] + g.reach[k];
    if (!g.pbc[k]) {
      lo[k] = lo[k] < 0 ? 0 : lo[k];
      hi[k] = hi[k] >= g.nb[k] ? g.nb[k] - 1 : hi[k];
    }
  }
  for (int bx = lo[0]; bx <= hi[0]; ++bx) {
    const int wx = ((bx % g.nb[0]) + g.nb[0]) % g.nb[0];
    const int sx = (bx - wx) / g.nb[0];
    for (int by = lo[1]; by <= hi[1]; ++by) {
      const int wy = ((by % g.nb[1]) + g.nb[1]) % g.nb[1];
      const int sy = (by - wy) / g.nb[1];
      for (int bz = lo[2]; bz <= hi[2]; ++bz) {
        const int wz = ((bz % g.nb[2]) + g.nb[2]) % g.nb[2];
        const int sz = (bz - wz) / g.nb[2];
        const int bl = b0 + (wx * g.nb[1] + wy) * g.nb[2] + wz;
        const int q1 = bstart[bl + 1];
        for (int q0 = bstart[bl]; q0 < q1; q0 += (WAVE ? 64 : 1)) {
          const int q = q0 + lane;
          int S[3] = {0, 0, 0};
          int b = 0;
          bool hit = false;
          if (q < q1) {
            b = batoms[q];
            hit = nl_pair(pos, aimg, g, a, ax, ay, az, oa, sx, sy, sz, b, S);
          }
          if (WAVE) {
            const unsigned long long m = __ballot(hit);
            if (FILL && hit) {
              const int slot = base + cnt + __popcll(m & ((1ull << lane) - 1ull));
              src[slot] = b;
              shift[3 * slot] = S[0];
              shift[3 * slot + 1] = S[1];
              shift[3 * slot + 2] = S[2];
            }
            cnt += __popcll(m);
          } else if (hit) {
            if (FILL) {
              const int slot = base + cnt;
              src[slot] = b;
              shift[3 * slot] = S[0];
              shift[3 * slot + 1] = S[1];
              shift[3 * slot + 2] = S[2];
            }
            ++cnt;
          }
        }
      }
    }
  }
  if (!FILL && lane == 0) counts[a] = cnt;
}

// --------------------------------------------------------------- C ABI --
extern "C" {

const char* tace_last_error(void) { return g_err; }

int tace_abi_version(void) { return TACE_HIP_ABI_VERSION; }

int tace_tp_num_variants(void) { return kNumVariants; }

const char* tace_tp_variant_key(int vid) {
  if (vid < 0 || vid >= kNumVariants) return nullptr;
  return kVariants[vid].key;
}

int tace_tp_find(const char* key) {
  if (!key) return fail("tace_tp_find: null key");
  for (int i = 0; i < kNumVariants; ++i)
    if (strcmp(kVariants[i].key, key) == 0) return i;
  snprintf(g_err, sizeof(g_err), "tace_tp_find: no compiled tensor-product variant for '%s'", key);
  return -1;
}

int tace_tp_dims(int vid, int32_t* npath, int32_t* d1, int32_t* d2, int32_t* dout) {
  if (vid < 0 || vid >= kNumVariants) return fail("tace_tp_dims: bad variant id");
  const TpVariant& v = kVariants[vid];
  if (npath) *npath = v.npath;
  if (d1) *d1 = v.d1;
  if (d2) *d2 = v.d2;
  if (dout) *dout = v.dout;
  return 0;
}

static int tp_common_checks(const char* who, int vid, int64_t n_nodes, int64_t n_edges, int32_t channels,
                            int32_t layout) {
  char msg[160];
  if (vid < 0 || vid >= kNumVariants || kVariants[vid].kind != 0) {
    snprintf(msg, sizeof(msg), "%s: bad variant id", who);
    return fail(msg);
  }
  if (layout < 0 || layout > 3) {
    snprintf(msg, sizeof(msg), "%s: layout must be a combination of IN1_GROUPED and OUT_GROUPED", who);
    return fail(msg);
  }
  if (channels <= 0 || channels > TACE_MAX_CHANNELS || n_nodes < 0 || n_edges < 0) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (channels must be in 1..%d)", who, TACE_MAX_CHANNELS);
    return fail(msg);
  }
  if (n_nodes > INT32_MAX || n_edges > INT32_MAX) {
    snprintf(msg, sizeof(msg), "%s: sizes exceed int32 indexing", who);
    return fail(msg);
  }
  return 0;
}

int tace_edge_tp_fwd_rows(int vid, int dtype, const void* x, const void* y, const void* w, const int32_t* rowptr,
                          const int32_t* eid, const int32_t* src, const int32_t* node_map, const int32_t* w_rows,
                          int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout, void* out,
                          void* stream) {
  if (tp_common_checks("tace_edge_tp_fwd", vid, n_nodes, n_edges, channels, layout)) return -1;
  if ((!x && n_edges) || (!out && n_nodes) || !rowptr || (n_edges && (!y || !w || !src)))
    return fail("tace_edge_tp_fwd: null pointer");
  const TpVariant& v = kVariants[vid];
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    v.fwd_f(x, y, w, rowptr, eid, src, node_map, w_rows, out, (int)n_nodes, layout, channels, s);
  else if (dtype == TACE_F64)
    v.fwd_d(x, y, w, rowptr, eid, src, node_map, w_rows, out, (int)n_nodes, layout, channels, s);
  else
    return fail("tace_edge_tp_fwd: dtype must be TACE_F32 or TACE_F64");
  return check_launch("tace_edge_tp_fwd");
}

int tace_edge_tp_fwd(int vid, int dtype, const void* x, const void* y, const void* w, const int32_t* rowptr,
                     const int32_t* eid, const int32_t* src, const int32_t* node_map, int64_t n_nodes, int64_t n_edges,
                     int32_t channels, int32_t layout, void* out, void* stream) {
  return tace_edge_tp_fwd_rows(vid, dtype, x, y, w, rowptr, eid, src, node_map, nullptr, n_nodes, n_edges, channels,
                               layout, out, stream);
}

// grad_y partials of one edge-TP backward launch: one per (part, channel
// group of 64); summed by k_sum_parts when there is more than one
static int tp_bwd_partials(const TpVariant& v, int channels) { return v.nparts * ((channels + 63) / 64); }

int64_t tace_edge_tp_workspace_elems(int vid, int64_t n_edges, int32_t channels, int32_t need_gx) {
  if (vid < 0 || vid >= kNumVariants || kVariants[vid].kind != 0) return fail("tace_edge_tp_workspace_elems: bad variant id");
  if (n_edges < 0 || channels <= 0) return fail("tace_edge_tp_workspace_elems: bad sizes");
  const TpVariant& v = kVariants[vid];
  int64_t n = need_gx ? n_edges * (int64_t)channels * v.d1 : 0;
  const int np = tp_bwd_partials(v, channels);
  if (np > 1) n += (int64_t)np * n_edges * v.d2;
  return n;
}

int tace_edge_tp_bwd(int vid, int dtype, const void* x, const void* y, const void* w, const void* gout,
                     const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                     int64_t n_nodes, int64_t n_edges,
                     int32_t channels, int32_t layout, const int32_t* s_rowptr, const int32_t* s_slot,
                     void* workspace, int64_t workspace_elems, void* gx, void* gy, void* gw, void* stream) {
  return tace_edge_tp_bwd_rows(vid, dtype, x, y, w, gout, rowptr, eid, src, node_map, nullptr, n_nodes, n_edges,
                               channels, layout, s_rowptr, s_slot, workspace, workspace_elems, gx, gy, gw, stream);
}

int tace_edge_tp_bwd_rows(int vid, int dtype, const void* x, const void* y, const void* w, const void* gout,
                          const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                          const int32_t* w_rows, int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                          const int32_t* s_rowptr, const int32_t* s_slot, void* workspace, int64_t workspace_elems,
                          void* gx, void* gy, void* gw, void* stream) {
  const hipEvent_t phase = g_phase_event;   // one-shot, cleared on every path
  g_phase_event = nullptr;
  if (tp_common_checks("tace_edge_tp_bwd", vid, n_nodes, n_edges, channels, layout)) return -1;
  if (!rowptr || (n_edges && (!x || !y || !w || !gout || !src || !gy || !gw)))
    return fail("tace_edge_tp_bwd: null pointer");
  const TpVariant& v = kVariants[vid];
  const int64_t row = (int64_t)channels * v.d1;
  const int64_t cb_elems = gx ? n_edges * row : 0;
  const int np = tp_bwd_partials(v, channels);
  if ((n_nodes + 7) / 8 * 8 * (int64_t)np > (int64_t)INT32_MAX)
    return fail("tace_edge_tp_bwd: too many receivers for one launch");
  const int64_t need = cb_elems + (np > 1 ? (int64_t)np * n_edges * v.d2 : 0);
  if (gx && !s_rowptr) return fail("tace_edge_tp_bwd: grad_x needs the sender CSR");
  if (n_edges && ((gx && !s_slot) || (need && !workspace))) return fail("tace_edge_tp_bwd: null sender CSR or workspace");
  if (workspace_elems < need) return fail("tace_edge_tp_bwd: workspace smaller than tace_edge_tp_workspace_elems()");
  RowSegs sg;
  memset(&sg, 0, sizeof(sg));
  if (layout & TACE_LAYOUT_IN1_GROUPED) {
    sg.n = v.nseg;
    for (int g = 0; g < v.nseg; ++g) {
      sg.off[g] = (int64_t)v.seg[g][0] * channels;
      sg.len[g] = (int64_t)v.seg[g][1] * channels;
    }
  }
  hipStream_t s = (hipStream_t)stream;
  if (dtype != TACE_F32 && dtype != TACE_F64) return fail("tace_edge_tp_bwd: dtype must be TACE_F32 or TACE_F64");
  const size_t es = dtype == TACE_F32 ? 4 : 8;
  // workspace = [grad_x rows of every slot | grad_y partial of every part]
  // cbuf == nullptr selects the kernels without grad_x
  void* cbuf = gx && n_edges ? workspace : nullptr;
  void* gyp = np > 1 ? (void*)((char*)workspace + cb_elems * es) : gy;
  const int64_t ny = n_edges * v.d2;
  const unsigned nb = (unsigned)((ny + 255) / 256);
  if (dtype == TACE_F32) {
    v.bwd_f(x, y, w, gout, rowptr, eid, src, node_map, w_rows, cbuf, gyp, gw, (int)n_nodes, (int)n_edges, layout,
            channels, s);
    if (phase) hipEventRecord(phase, s);
    if (np > 1 && ny)
      sum_parts_f32((const float*)gyp, np, ny, (float*)gy, 0, s);
    if (gx && n_nodes)
      launch_seg_rowsum<float>((const float*)cbuf, s_rowptr, s_slot, node_map, (float*)gx, (int)n_nodes, row, sg,
                               channels, s);
  } else {
    v.bwd_d(x, y, w, gout, rowptr, eid, src, node_map, w_rows, cbuf, gyp, gw, (int)n_nodes, (int)n_edges, layout,
            channels, s);
    if (phase) hipEventRecord(phase, s);
    if (np > 1 && ny)
      hipLaunchKernelGGL(k_sum_parts<double>, dim3(nb), dim3(256), 0, s, (const double*)gyp, np, ny,
                         (double*)gy);
    if (gx && n_nodes)
      launch_seg_rowsum<double>((const double*)cbuf, s_rowptr, s_slot, node_map, (double*)gx, (int)n_nodes, row, sg,
                                channels, s);
  }
  return check_launch("tace_edge_tp_bwd");
}

// ------------------------------------------ allocation-free edge-TP backward --
// The workspace of tace_edge_tp_bwd (per-slot grad_x rows and per-part grad_y
// partials) taken from a file-scope device array instead of a caller buffer.
// Each GPU holds its own copy of `scratch` for the life of the process; host
// code never uses the array's name as an address: the per-device address
// comes from hipGetSymbolAddress once per device (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[TACE_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[TACE_NOALLOC_MAX_DEVICES];

// address of the current device's `scratch`, looked up on the first call per
// device (with that device current) and kept; nullptr after fail()
static void* noalloc_scratch(const char* who) {
  char msg[200];
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= TACE_NOALLOC_MAX_DEVICES) {
    snprintf(msg, sizeof(msg), "%s: no usable current device (%s)", who,
             e != hipSuccess ? hipGetErrorString(e) : "device index out of range");
    fail(msg);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      snprintf(msg, sizeof(msg), "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
               hipGetErrorString(e));
      fail(msg);
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

int tace_edge_tp_bwd_noalloc(int vid, int dtype, const void* x, const void* y, const void* w, const void* gout,
                             const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                             int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                             const int32_t* s_rowptr, const int32_t* s_slot, void* gx, void* gy, void* gw,
                             void* stream) {
  if (tp_common_checks("tace_edge_tp_bwd_noalloc", vid, n_nodes, n_edges, channels, layout)) return -1;
  if (dtype != TACE_F32 && dtype != TACE_F64)
    return fail("tace_edge_tp_bwd_noalloc: dtype must be TACE_F32 or TACE_F64");
  const int64_t elems = tace_edge_tp_workspace_elems(vid, n_edges, channels, gx != nullptr);
  if (elems < 0) return -1;
  const int64_t es = dtype == TACE_F32 ? 4 : 8;
  if (elems > TACE_NOALLOC_SCRATCH_BYTES / es) {
    char msg[240];
    snprintf(msg, sizeof(msg),
             "tace_edge_tp_bwd_noalloc: needs %lld bytes of scratch (E=%lld, C=%d), above the %lld-byte maximum; "
             "use tace_edge_tp_bwd with a caller workspace",
             (long long)(elems * es), (long long)n_edges, (int)channels, (long long)TACE_NOALLOC_SCRATCH_BYTES);
    return fail(msg);
  }
  void* ws = nullptr;
  if (elems > 0 && !(ws = noalloc_scratch("tace_edge_tp_bwd_noalloc"))) return -1;
  // every scratch element the kernels read is written earlier in the same
  // call (all grad_x row segments of every slot by the parts, every grad_y
  // partial), so nothing needs clearing between calls
  return tace_edge_tp_bwd(vid, dtype, x, y, w, gout, rowptr, eid, src, node_map, n_nodes, n_edges, channels, layout,
                          s_rowptr, s_slot, ws, elems, gx, gy, gw, stream);
}

// ---------------------------------------------- radial-fused edge products --
// Receivers per persistent workgroup: about 2048 workgroups in all (8 per CU
// over the launch), at least one receiver each.
static int rtp_per_range(int64_t n_nodes, int nph) {
  const int64_t ranges = 2048 / nph > 8 ? 2048 / nph : 8;
  const int64_t per = (n_nodes + ranges - 1) / ranges;
  return per > 0 ? (int)per : 1;
}

// slot_rows[k] = feature row of the sender of receiver-sorted slot k
__global__ __launch_bounds__(256) void k_slot_rows(const int32_t* __restrict__ eid, const int32_t* __restrict__ src,
                                                   const int32_t* __restrict__ node_map, int64_t E,
                                                   int32_t* __restrict__ out) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= E) return;
  const int32_t s = src[eid ? eid[k] : k];
  out[k] = node_map ? node_map[s] : s;
}

static void launch_slot_rows(const int32_t* eid, const int32_t* src, const int32_t* node_map, int64_t E, int32_t* out,
                             hipStream_t s) {
  if (E > 0)
    hipLaunchKernelGGL(k_slot_rows, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, s, eid, src, node_map, E, out);
}

static int rtp_checks(const char* who, int vid, int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                      const float* h) {
  char msg[200];
  if (tp_common_checks(who, vid, n_nodes, n_edges, channels, layout)) return -1;
  if (!kVariants[vid].rfwd) {
    snprintf(msg, sizeof(msg), "%s: variant %s has no radial-fused kernels", who, kVariants[vid].key);
    return fail(msg);
  }
  if (channels % 64 != 0) {
    snprintf(msg, sizeof(msg), "%s: channels must be a multiple of 64 (got %d)", who, (int)channels);
    return fail(msg);
  }
  if (((uintptr_t)h & 15) != 0) {
    snprintf(msg, sizeof(msg), "%s: h must be 16-byte aligned", who);
    return fail(msg);
  }
  return 0;
}

int tace_edge_rtp_fwd(int vid, const float* x, const float* y, const float* h, const float* w_last, float alpha,
                      const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                      int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout, int32_t* slot_rows,
                      float* out, void* stream) {
  if (rtp_checks("tace_edge_rtp_fwd", vid, n_nodes, n_edges, channels, layout, h)) return -1;
  if ((!out && n_nodes) || !rowptr || !w_last || (n_edges && (!x || !y || !h || !src || !slot_rows)))
    return fail("tace_edge_rtp_fwd: null pointer");
  const TpVariant& v = kVariants[vid];
  const int nph = v.rnparts * (channels / 64);
  hipStream_t s = (hipStream_t)stream;
  launch_slot_rows(eid, src, node_map, n_edges, slot_rows, s);
  v.rfwd(x, y, h, w_last, alpha, rowptr, eid, src, node_map, slot_rows, out, (int)n_nodes, layout, channels,
         rtp_per_range(n_nodes, nph), s);
  return check_launch("tace_edge_rtp_fwd");
}

int64_t tace_edge_rtp_workspace_elems(int vid, int64_t n_edges, int32_t channels, int32_t need_gx) {
  if (vid < 0 || vid >= kNumVariants || kVariants[vid].kind != 0 || !kVariants[vid].rfwd)
    return fail("tace_edge_rtp_workspace_elems: bad variant id");
  if (n_edges < 0 || channels <= 0 || channels % 64 != 0) return fail("tace_edge_rtp_workspace_elems: bad sizes");
  const TpVariant& v = kVariants[vid];
  const int64_t nph = (int64_t)v.rnparts * (channels / 64);
  int64_t n = need_gx ? n_edges * (int64_t)channels * v.d1 : 0;
  if (nph > 1) n += nph * n_edges * v.d2;
  return n;
}

int tace_edge_rtp_bwd(int vid, const float* x, const float* y, const float* h, const float* w_last, float alpha,
                      const float* gout, const int32_t* rowptr, const int32_t* eid, const int32_t* src,
                      const int32_t* node_map, int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                      const int32_t* s_rowptr, const int32_t* s_slot, int32_t* slot_rows, float* workspace,
                      int64_t workspace_elems, float* gx, float* gy, float* gw, void* stream) {
  if (rtp_checks("tace_edge_rtp_bwd", vid, n_nodes, n_edges, channels, layout, h)) return -1;
  if (!rowptr || !w_last || (n_edges && (!x || !y || !h || !gout || !src || !gy || !gw || !slot_rows)))
    return fail("tace_edge_rtp_bwd: null pointer");
  const TpVariant& v = kVariants[vid];
  const int nph = v.rnparts * (channels / 64);
  const int64_t row = (int64_t)channels * v.d1;
  const int64_t cb_elems = gx ? n_edges * row : 0;
  const int64_t need = cb_elems + (nph > 1 ? (int64_t)nph * n_edges * v.d2 : 0);
  if (gx && !s_rowptr) return fail("tace_edge_rtp_bwd: grad_x needs the sender CSR");
  if (n_edges && ((gx && !s_slot) || (need && !workspace)))
    return fail("tace_edge_rtp_bwd: null sender CSR or workspace");
  if (workspace_elems < need) return fail("tace_edge_rtp_bwd: workspace smaller than tace_edge_rtp_workspace_elems()");
  RowSegs sg;
  memset(&sg, 0, sizeof(sg));
  if (layout & TACE_LAYOUT_IN1_GROUPED) {
    sg.n = v.nseg;
    for (int g = 0; g < v.nseg; ++g) {
      sg.off[g] = (int64_t)v.seg[g][0] * channels;
      sg.len[g] = (int64_t)v.seg[g][1] * channels;
    }
  }
  hipStream_t s = (hipStream_t)stream;
  // workspace = [grad_x rows of every slot | grad_y partial of every (part, 64 channels)]
  float* cbuf = gx && n_edges ? workspace : nullptr;
  float* gyp = nph > 1 ? workspace + cb_elems : gy;
  const int64_t ny = n_edges * v.d2;
  launch_slot_rows(eid, src, node_map, n_edges, slot_rows, s);
  v.rbwd(x, y, h, w_last, alpha, gout, rowptr, eid, src, node_map, slot_rows, cbuf, gyp, gw, (int)n_nodes,
         (int)n_edges, layout, channels, rtp_per_range(n_nodes, nph), s);
  if (nph > 1 && ny)
    sum_parts_f32((const float*)gyp, nph, ny, gy, 0, s);
  if (gx && n_nodes)
    launch_seg_rowsum<float>(cbuf, s_rowptr, s_slot, node_map, gx, (int)n_nodes, row, sg, channels, s);
  return check_launch("tace_edge_rtp_bwd");
}

static bool uuu_layout_ok(int32_t layout) {
  return layout == 0 || layout == TACE_LAYOUT_OUT_GROUPED ||
         layout == (TACE_LAYOUT_IN1_GROUPED | TACE_LAYOUT_OUT_GROUPED) ||
         layout == (TACE_LAYOUT_IN1_GROUPED | TACE_LAYOUT_OUT_GROUPED | TACE_LAYOUT_IN2_GROUPED);
}

int tace_uuu_fwd(int vid, int dtype, const void* x1, const void* x2, const void* w, int64_t n_nodes, int32_t channels,
                 int32_t layout, void* out, void* stream) {
  if (vid < 0 || vid >= kNumVariants || kVariants[vid].kind != 1) return fail("tace_uuu_fwd: bad variant id");
  if (channels <= 0 || n_nodes < 0) return fail("tace_uuu_fwd: bad sizes");
  if (!uuu_layout_ok(layout)) return fail("tace_uuu_fwd: layout must be 0, OUT, IN1|OUT or IN1|OUT|IN2 (GROUPED)");
  if (n_nodes && (!x1 || !x2 || !out)) return fail("tace_uuu_fwd: null pointer");
  if ((size_t)n_nodes * channels > (size_t)UINT32_MAX * 128) return fail("tace_uuu_fwd: too many nodes");
  const TpVariant& v = kVariants[vid];
  if (n_nodes && v.weighted != (w != nullptr))
    return fail(v.weighted ? "tace_uuu_fwd: this product is weighted: w is required"
                           : "tace_uuu_fwd: this product has no path weights: w must be null");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    v.ufwd_f(x1, x2, w, out, (int)n_nodes, channels, layout, s);
  else if (dtype == TACE_F64)
    v.ufwd_d(x1, x2, w, out, (int)n_nodes, channels, layout, s);
  else
    return fail("tace_uuu_fwd: dtype must be TACE_F32 or TACE_F64");
  return check_launch("tace_uuu_fwd");
}

// Workspace of the backward: grad_x2 partials when there are several parts
// or when grad_x2 is added to g2 (accumulate bit 1), then grad_x1 when it is
// added to g1 (bit 0); the sums into g1 / g2 run after the product kernel.
static int64_t uuu_ws_g1_offset(const TpVariant& v, int64_t n_nodes, int32_t channels, int32_t accumulate) {
  return (v.unparts > 1 || (accumulate & 2)) ? (int64_t)v.unparts * n_nodes * channels * v.d2 : 0;
}

static int64_t uuu_ws_elems(const TpVariant& v, int64_t n_nodes, int32_t channels, int32_t accumulate) {
  return uuu_ws_g1_offset(v, n_nodes, channels, accumulate) +
         ((accumulate & 1) ? n_nodes * (int64_t)channels * v.d1 : 0);
}

int64_t tace_uuu_workspace_elems(int vid, int64_t n_nodes, int32_t channels, int32_t accumulate) {
  if (vid < 0 || vid >= kNumVariants || kVariants[vid].kind != 1) return fail("tace_uuu_workspace_elems: bad variant id");
  if (channels <= 0 || n_nodes < 0) return fail("tace_uuu_workspace_elems: bad sizes");
  if (accumulate & ~3) return fail("tace_uuu_workspace_elems: accumulate takes bits 0 and 1 only");
  return uuu_ws_elems(kVariants[vid], n_nodes, channels, accumulate);
}

int tace_uuu_bwd(int vid, int dtype, const void* x1, const void* x2, const void* w, const void* gout, int64_t n_nodes,
                 int32_t channels, int32_t layout, void* g1, void* g2, void* gw, void* workspace,
                 int64_t workspace_elems, int32_t accumulate, void* stream) {
  if (vid < 0 || vid >= kNumVariants || kVariants[vid].kind != 1) return fail("tace_uuu_bwd: bad variant id");
  if (channels <= 0 || n_nodes < 0) return fail("tace_uuu_bwd: bad sizes");
  if (!uuu_layout_ok(layout)) return fail("tace_uuu_bwd: layout must be 0, OUT, IN1|OUT or IN1|OUT|IN2 (GROUPED)");
  if (n_nodes && (!x1 || !x2 || !gout || !g1 || !g2)) return fail("tace_uuu_bwd: null pointer");
  const TpVariant& v = kVariants[vid];
  if (((size_t)n_nodes * channels + 255) / 256 * v.unparts > (size_t)UINT32_MAX) return fail("tace_uuu_bwd: too many nodes");
  if (n_nodes && v.weighted != (w != nullptr))
    return fail(v.weighted ? "tace_uuu_bwd: this product is weighted: w is required"
                           : "tace_uuu_bwd: this product has no path weights: w must be null");
  if (n_nodes && w && !gw) return fail("tace_uuu_bwd: weighted products need gw");
  if (accumulate & ~3) return fail("tace_uuu_bwd: accumulate takes bits 0 and 1 only");
  if (g1 == g2 && n_nodes &&
      (accumulate != 3 || !(layout & TACE_LAYOUT_IN1_GROUPED) != !(layout & TACE_LAYOUT_IN2_GROUPED) || v.d1 != v.d2))
    return fail("tace_uuu_bwd: g1 and g2 may be one array only when both accumulate into it, in one layout");
  const int64_t ny = n_nodes * (int64_t)channels * v.d2;
  const int64_t need = uuu_ws_elems(v, n_nodes, channels, accumulate);
  if (need && !workspace) return fail("tace_uuu_bwd: null workspace");
  if (workspace_elems < need) return fail("tace_uuu_bwd: workspace smaller than tace_uuu_workspace_elems()");
  hipStream_t s = (hipStream_t)stream;
  // parts > 1 (or grad_x2 accumulated): each part writes its grad_x2 partial
  // into the workspace, and the partials are summed into g2 in a fixed order;
  // grad_x1 accumulated: the kernel writes it into the workspace too, and it
  // is added to g1 first (so g1 == g2 receives grad_x1, then grad_x2)
  const int64_t off1 = uuu_ws_g1_offset(v, n_nodes, channels, accumulate);
  const bool ws2 = off1 > 0;
  const int acc1 = accumulate & 1, acc2 = (accumulate >> 1) & 1;
  const int64_t n1 = n_nodes * (int64_t)channels * v.d1;
  const unsigned nb = (unsigned)((ny + 255) / 256), nb1 = (unsigned)((n1 + 255) / 256);
  if (dtype == TACE_F32) {
    float* wsf = (float*)workspace;
    void* g1k = acc1 ? (void*)(wsf + off1) : g1;
    void* g2p = ws2 ? workspace : g2;
    v.ubwd_f(x1, x2, w, gout, g1k, g2p, w ? gw : nullptr, (int)n_nodes, channels, layout, s);
    if (acc1 && n1)
      sum_parts_f32((const float*)g1k, 1, n1, (float*)g1, 1, s);
    if (ws2 && ny)
      sum_parts_f32((const float*)g2p, v.unparts, ny, (float*)g2, acc2, s);
  } else if (dtype == TACE_F64) {
    double* wsd = (double*)workspace;
    void* g1k = acc1 ? (void*)(wsd + off1) : g1;
    void* g2p = ws2 ? workspace : g2;
    v.ubwd_d(x1, x2, w, gout, g1k, g2p, w ? gw : nullptr, (int)n_nodes, channels, layout, s);
    if (acc1 && n1)
      hipLaunchKernelGGL(k_sum_parts<double>, dim3(nb1), dim3(256), 0, s, (const double*)g1k, 1, n1, (double*)g1, 1);
    if (ws2 && ny)
      hipLaunchKernelGGL(k_sum_parts<double>, dim3(nb), dim3(256), 0, s, (const double*)g2p, v.unparts, ny,
                         (double*)g2, acc2);
  } else {
    return fail("tace_uuu_bwd: dtype must be TACE_F32 or TACE_F64");
  }
  return check_launch("tace_uuu_bwd");
}

int tace_edge_basis_fwd(int dtype, const void* vec, int64_t n_edges, int32_t num_basis, const void* bessel_w,
                        double prefactor, double cutoff, int32_t poly_p, int32_t lmax, void* radial, void* sh,
                        void* stream) {
  if (n_edges < 0 || num_basis <= 0 || poly_p < 1) return fail("tace_edge_basis_fwd: bad sizes");
  if (n_edges && (!vec || !bessel_w || !radial || !sh)) return fail("tace_edge_basis_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    return edge_basis_fwd_t<float>((const float*)vec, n_edges, num_basis, (const float*)bessel_w, prefactor, cutoff,
                                   poly_p, lmax, (float*)radial, (float*)sh, s);
  if (dtype == TACE_F64)
    return edge_basis_fwd_t<double>((const double*)vec, n_edges, num_basis, (const double*)bessel_w, prefactor, cutoff,
                                    poly_p, lmax, (double*)radial, (double*)sh, s);
  return fail("tace_edge_basis_fwd: dtype must be TACE_F32 or TACE_F64");
}

int tace_edge_basis_bwd(int dtype, const void* vec, const void* g_radial, const void* g_sh, int64_t n_edges,
                        int32_t num_basis, const void* bessel_w, double prefactor, double cutoff, int32_t poly_p,
                        int32_t lmax, void* g_vec, void* stream) {
  if (n_edges < 0 || num_basis <= 0 || poly_p < 1) return fail("tace_edge_basis_bwd: bad sizes");
  if (n_edges && (!vec || !g_radial || !g_sh || !bessel_w || !g_vec)) return fail("tace_edge_basis_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    return edge_basis_bwd_t<float>((const float*)vec, (const float*)g_radial, (const float*)g_sh, n_edges, num_basis,
                                   (const float*)bessel_w, prefactor, cutoff, poly_p, lmax, (float*)g_vec, s);
  if (dtype == TACE_F64)
    return edge_basis_bwd_t<double>((const double*)vec, (const double*)g_radial, (const double*)g_sh, n_edges,
                                    num_basis, (const double*)bessel_w, prefactor, cutoff, poly_p, lmax,
                                    (double*)g_vec, s);
  return fail("tace_edge_basis_bwd: dtype must be TACE_F32 or TACE_F64");
}

int tace_edge_vec_fwd(int dtype, const void* pos, const void* lattice, const int32_t* src, const int32_t* dst,
                      const void* shifts, const int32_t* edge_graph, int64_t n_edges, void* vec, void* stream) {
  if (n_edges < 0) return fail("tace_edge_vec_fwd: bad sizes");
  if (n_edges == 0) return 0;
  if (!pos || !lattice || !src || !dst || !shifts || !vec) return fail("tace_edge_vec_fwd: null pointer");
  const dim3 g((unsigned)((n_edges + 255) / 256)), b(256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_edge_vec_fwd<float>, g, b, 0, s, (const float*)pos, (const float*)lattice, src, dst,
                       (const float*)shifts, edge_graph, n_edges, (float*)vec);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_edge_vec_fwd<double>, g, b, 0, s, (const double*)pos, (const double*)lattice, src, dst,
                       (const double*)shifts, edge_graph, n_edges, (double*)vec);
  else
    return fail("tace_edge_vec_fwd: dtype must be TACE_F32 or TACE_F64");
  return check_launch("tace_edge_vec_fwd");
}

int tace_edge_vec_bwd(int dtype, const void* g_vec, const int32_t* rowptr, const int32_t* eid,
                      const int32_t* s_rowptr, const int32_t* s_slot, int64_t n_nodes, void* g_pos, void* stream) {
  if (n_nodes < 0 || n_nodes > INT32_MAX) return fail("tace_edge_vec_bwd: bad sizes");
  if (n_nodes == 0) return 0;
  if (!g_vec || !rowptr || !s_rowptr || !s_slot || !g_pos) return fail("tace_edge_vec_bwd: null pointer");
  const dim3 g((unsigned)((n_nodes + 255) / 256)), b(256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_edge_vec_bwd<float>, g, b, 0, s, (const float*)g_vec, rowptr, eid, s_rowptr, s_slot,
                       (int)n_nodes, (float*)g_pos);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_edge_vec_bwd<double>, g, b, 0, s, (const double*)g_vec, rowptr, eid, s_rowptr, s_slot,
                       (int)n_nodes, (double*)g_pos);
  else
    return fail("tace_edge_vec_bwd: dtype must be TACE_F32 or TACE_F64");
  return check_launch("tace_edge_vec_bwd");
}

int64_t tace_nl_workspace_bytes(int64_t n_atoms, const double* cell, const int32_t* pbc, double cutoff) {
  NlGeom g;
  if (!cell || !pbc) return fail("tace_nl_workspace_bytes: null pointer");
  if (nl_geometry(cell, pbc, cutoff, &g)) return -1;
  const int64_t nbins = (int64_t)g.nb[0] * g.nb[1] * g.nb[2];
  // abin[n], aimg[3n], bcount[nbins], bstart[nbins+1], bfill[nbins], batoms[n],
  // unsorted[n] (the bin contents before the ranking; tace_nl_count only)
  return (int64_t)sizeof(int32_t) * (n_atoms * 6 + nbins * 3 + 1);
}

int tace_nl_count(const double* pos, int64_t n_atoms, const double* cell, const int32_t* pbc, double cutoff,
                  void* workspace, int64_t workspace_bytes, int32_t* counts, void* stream) {
  NlGeom g;
  if (!cell || !pbc) return fail("tace_nl_count: null pointer");
  if (nl_geometry(cell, pbc, cutoff, &g)) return -1;
  if (n_atoms < 0 || n_atoms > INT32_MAX / 8) return fail("tace_nl_count: bad atom count");
  if (n_atoms == 0) return 0;
  if (!pos || !workspace || !counts) return fail("tace_nl_count: null pointer");
  const int64_t nbins = (int64_t)g.nb[0] * g.nb[1] * g.nb[2];
  if (workspace_bytes < (int64_t)sizeof(int32_t) * (n_atoms * 6 + nbins * 3 + 1))
    return fail("tace_nl_count: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const int n = (int)n_atoms;
  int* abin = (int*)workspace;
  int* aimg = abin + n;
  int* bcount = aimg + 3 * n;
  int* bstart = bcount + nbins;
  int* bfill = bstart + nbins + 1;
  int* batoms = bfill + nbins;
  int* unsorted = batoms + n;
  launch_fill<int>(bcount, (size_t)nbins, 0, s);
  launch_fill<int>(bfill, (size_t)nbins, 0, s);
  const dim3 ga((n + 255) / 256), ba(256);
  hipLaunchKernelGGL(k_nl_bin, ga, ba, 0, s, pos, n, g, abin, aimg, bcount);
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, s, bcount, (int)nbins, bstart);
  hipLaunchKernelGGL(k_nl_scatter, ga, ba, 0, s, abin, n, bstart, bfill, unsorted);
  hipLaunchKernelGGL(k_nlb_rank, ga, ba, 0, s, abin, n, bstart, unsorted, batoms);
  if (n < NL_WAVE_MAX)
    hipLaunchKernelGGL((k_nl_edges<false, true>), dim3((n + 3) / 4), dim3(256), 0, s, pos, n, g, abin, aimg, bstart,
                       batoms, counts, nullptr, nullptr, nullptr);
  else
    hipLaunchKernelGGL((k_nl_edges<false, false>), dim3((n + 255) / 256), dim3(256), 0, s, pos, n, g, abin, aimg,
                       bstart, batoms, counts, nullptr, nullptr, nullptr);
  return check_launch("tace_nl_count");
}

int tace_nl_fill(const double* pos, int64_t n_atoms, const double* cell, const int32_t* pbc, double cutoff,
                 const void* workspace, const int32_t* rowptr, int32_t* src, int32_t* shifts, void* stream) {
  NlGeom g;
  if (!cell || !pbc) return fail("tace_nl_fill: null pointer");
  if (nl_geometry(cell, pbc, cutoff, &g)) return -1;
  if (n_atoms <= 0) return 0;
  if (!pos || !workspace || !rowptr || !src || !shifts) return fail("tace_nl_fill: null pointer");
  const int64_t nbins = (int64_t)g.nb[0] * g.nb[1] * g.nb[2];
  hipStream_t s = (hipStream_t)stream;
  const int n = (int)n_atoms;
  const int* abin = (const int*)workspace;
  const int* aimg = abin + n;
  const int* bcount = aimg + 3 * n;
  const int* bstart = bcount + nbins;
  const int* bfill = bstart + nbins + 1;
  const int* batoms = bfill + nbins;
  if (n < NL_WAVE_MAX)
    hipLaunchKernelGGL((k_nl_edges<true, true>), dim3((n + 3) / 4), dim3(256), 0, s, pos, n, g, abin, aimg, bstart,
                       batoms, nullptr, rowptr, src, shifts);
  else
    hipLaunchKernelGGL((k_nl_edges<true, false>), dim3((n + 255) / 256), dim3(256), 0, s, pos, n, g, abin, aimg,
                       bstart, batoms, nullptr, rowptr, src, shifts);
  return check_launch("tace_nl_fill");
}

// plan table: NlGeom[ns], then int32 struct_ptr[ns+1], int32 bin_off[ns+1]
static int64_t nlb_plan_bytes(int64_t ns) {
  return (int64_t)sizeof(NlGeom) * ns + (int64_t)sizeof(int32_t) * 2 * (ns + 1);
}

int64_t tace_nl_batch_plan(int32_t n_structs, const int64_t* sizes, const double* cells, const int32_t* pbcs,
                           double cutoff, void* plan, int64_t plan_bytes, int64_t* n_atoms, int64_t* n_bins) {
  if (n_structs < 1) return fail("tace_nl_batch_plan: need at least one structure");
  if (!sizes || !cells || !pbcs || !n_atoms || !n_bins) return fail("tace_nl_batch_plan: null pointer");
  const int64_t need = nlb_plan_bytes(n_structs);
  if (!plan) return need;
  if (plan_bytes < need) return fail("tace_nl_batch_plan: plan buffer too small");
  NlGeom* geo = (NlGeom*)plan;
  int32_t* sptr = (int32_t*)(geo + n_structs);
  int32_t* boff = sptr + n_structs + 1;
  int64_t na = 0, nb = 0;
  for (int32_t i = 0; i < n_structs; ++i) {
    if (sizes[i] < 0) return fail("tace_nl_batch_plan: negative structure size");
    if (nl_geometry(cells + 9 * (int64_t)i, pbcs + 3 * (int64_t)i, cutoff, geo + i)) return -1;
    sptr[i] = (int32_t)na;
    boff[i] = (int32_t)nb;
    na += sizes[i];
    nb += (int64_t)geo[i].nb[0] * geo[i].nb[1] * geo[i].nb[2];
    if (na > INT32_MAX / 8 || nb > INT32_MAX / 8) return fail("tace_nl_batch_plan: batch too large");
  }
  sptr[n_structs] = (int32_t)na;
  boff[n_structs] = (int32_t)nb;
  *n_atoms = na;
  *n_bins = nb;
  return need;
}

int64_t tace_nl_batch_workspace_bytes(int64_t n_atoms, int64_t n_bins) {
  if (n_atoms < 0 || n_bins < 0 || n_atoms > INT32_MAX / 8 || n_bins > INT32_MAX / 8)
    return fail("tace_nl_batch_workspace_bytes: bad sizes");
  return (int64_t)sizeof(int32_t) * (n_atoms * 6 + n_bins * 3 + 1);
}

static int nlb_setup(const char* what, const void* plan, int32_t n_structs, int64_t n_atoms, int64_t n_bins,
                     const void* workspace, int64_t workspace_bytes, NlBatch* B) {
  if (n_structs < 1 || n_atoms < 0 || n_bins < 1 || n_atoms > INT32_MAX / 8 || n_bins > INT32_MAX / 8) {
    char m[160];
    snprintf(m, sizeof m, "%s: bad sizes", what);
    return fail(m);
  }
  if (!plan || !workspace) {
    char m[160];
    snprintf(m, sizeof m, "%s: null pointer", what);
    return fail(m);
  }
  if (workspace_bytes < (int64_t)sizeof(int32_t) * (n_atoms * 6 + n_bins * 3 + 1)) {
    char m[160];
    snprintf(m, sizeof m, "%s: workspace too small", what);
    return fail(m);
  }
  B->geo = (const NlGeom*)plan;
  B->sptr = (const int*)(B->geo + n_structs);
  B->boff = B->sptr + n_structs + 1;
  B->ns = n_structs;
  return 0;
}

static bool nlb_wave_mode(int64_t n_atoms, int32_t mode) {
  return mode == 2 || (mode == 0 && n_atoms < 32768);
}

int tace_nl_batch_count(const double* pos, int64_t n_atoms, int32_t n_structs, const void* plan, int64_t n_bins,
                        void* workspace, int64_t workspace_bytes, int32_t mode, int32_t* counts, void* stream) {
  NlBatch B;
  if (nlb_setup("tace_nl_batch_count", plan, n_structs, n_atoms, n_bins, workspace, workspace_bytes, &B)) return -1;
  if (mode < 0 || mode > 2) return fail("tace_nl_batch_count: mode must be 0 (auto), 1 (thread) or 2 (wave)");
  if (n_atoms == 0) return 0;
  if (!pos || !counts) return fail("tace_nl_batch_count: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int n = (int)n_atoms, nb = (int)n_bins;
  int* abin = (int*)workspace;
  int* aimg = abin + n;
  int* bcount = aimg + 3 * n;
  int* bstart = bcount + nb;
  int* bfill = bstart + nb + 1;
  int* batoms = bfill + nb;
  int* unsorted = batoms + n;
  launch_fill<int>(bcount, (size_t)nb, 0, s);
  launch_fill<int>(bfill, (size_t)nb, 0, s);
  const dim3 ga((n + 255) / 256), ba(256);
  hipLaunchKernelGGL(k_nlb_bin, ga, ba, 0, s, pos, n, B, abin, aimg, bcount);
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, s, bcount, nb, bstart);
  hipLaunchKernelGGL(k_nl_scatter, ga, ba, 0, s, abin, n, bstart, bfill, unsorted);
  hipLaunchKernelGGL(k_nlb_rank, ga, ba, 0, s, abin, n, bstart, unsorted, batoms);
  if (nlb_wave_mode(n_atoms, mode))
    hipLaunchKernelGGL((k_nlb_edges<false, true>), dim3((n + 3) / 4), dim3(256), 0, s, pos, n, B, abin, aimg,
                       bstart, batoms, counts, nullptr, nullptr, nullptr);
  else
    hipLaunchKernelGGL((k_nlb_edges<false, false>), dim3((n + 255) / 256), dim3(256), 0, s, pos, n, B, abin, aimg,
                       bstart, batoms, counts, nullptr, nullptr, nullptr);
  return check_launch("tace_nl_batch_count");
}

int tace_nl_batch_fill(const double* pos, int64_t n_atoms, int32_t n_structs, const void* plan, int64_t n_bins,
                       const void* workspace, int64_t workspace_bytes, int32_t mode, const int32_t* rowptr,
                       int32_t* src, int32_t* shifts, void* stream) {
  NlBatch B;
  if (nlb_setup("tace_nl_batch_fill", plan, n_structs, n_atoms, n_bins, workspace, workspace_bytes, &B)) return -1;
  if (mode < 0 || mode > 2) return fail("tace_nl_batch_fill: mode must be 0 (auto), 1 (thread) or 2 (wave)");
  if (n_atoms == 0) return 0;
  if (!pos || !rowptr || !src || !shifts) return fail("tace_nl_batch_fill: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int n = (int)n_atoms, nb = (int)n_bins;
  const int* abin = (const int*)workspace;
  const int* aimg = abin + n;
  const int* bcount = aimg + 3 * n;
  const int* bstart = bcount + nb;
  const int* bfill = bstart + nb + 1;
  const int* batoms = bfill + nb;
  if (nlb_wave_mode(n_atoms, mode))
    hipLaunchKernelGGL((k_nlb_edges<true, true>), dim3((n + 3) / 4), dim3(256), 0, s, pos, n, B, abin, aimg,
                       bstart, batoms, nullptr, rowptr, src, shifts);
  else
    hipLaunchKernelGGL((k_nlb_edges<true, false>), dim3((n + 255) / 256), dim3(256), 0, s, pos, n, B, abin, aimg,
                       bstart, batoms, nullptr, rowptr, src, shifts);
  return check_launch("tace_nl_batch_fill");
}

static int rows_accumulate(int dtype, const void* rows, int64_t n_rows, int64_t width, const int32_t* rowptr,
                           const int32_t* slot, const int32_t* target, int64_t n_segments, int32_t run, void* out,
                           int64_t n_out_rows, void* stream);

int tace_rows_accumulate(int dtype, const void* rows, int64_t n_rows, int64_t width, const int32_t* rowptr,
                         const int32_t* slot, const int32_t* target, int64_t n_segments, void* out,
                         int64_t n_out_rows, void* stream) {
  return rows_accumulate(dtype, rows, n_rows, width, rowptr, slot, target, n_segments, 1, out, n_out_rows, stream);
}

int tace_narrow_linear(int dtype, const void* x, int64_t n_rows, int32_t k, const void* m, const void* bias,
                       int32_t n, void* out, void* stream) {
  if (n_rows < 0 || k <= 0 || k > 64 || n <= 0 || n > 64) return fail("tace_narrow_linear: bad sizes (k, n in 1..64)");
  if (n_rows == 0) return 0;
  if (!x || !m || !out) return fail("tace_narrow_linear: null pointer");
  if (n_rows * n / 256 + 1 > (int64_t)UINT32_MAX) return fail("tace_narrow_linear: too many rows");
  const dim3 g((unsigned)((n_rows * n + 255) / 256)), b(256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_narrow_linear<float>, g, b, 0, s, (const float*)x, n_rows, (int)k, (const float*)m,
                       (const float*)bias, (int)n, (float*)out);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_narrow_linear<double>, g, b, 0, s, (const double*)x, n_rows, (int)k, (const double*)m,
                       (const double*)bias, (int)n, (double*)out);
  else
    return fail("tace_narrow_linear: dtype must be TACE_F32 or TACE_F64");
  return check_launch("tace_narrow_linear");
}

int tace_graph_sum(int dtype, const void* values, int64_t n_rows, int64_t width, const int64_t* ptr,
                   int64_t n_graphs, void* out, void* stream) {
  if (n_rows < 0 || width <= 0 || width > 4096 || n_graphs < 0 || n_graphs > INT32_MAX)
    return fail("tace_graph_sum: bad sizes (0 < width <= 4096)");
  if (n_graphs == 0) return 0;
  if (!ptr || !out || (n_rows > 0 && !values)) return fail("tace_graph_sum: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_graph_sum<float>, dim3((unsigned)n_graphs), dim3(256), 0, s, (const float*)values, width, ptr,
                       (float*)out);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_graph_sum<double>, dim3((unsigned)n_graphs), dim3(256), 0, s, (const double*)values, width,
                       ptr, (double*)out);
  else
    return fail("tace_graph_sum: dtype must be TACE_F32 or TACE_F64");
  return check_launch("tace_graph_sum");
}

int tace_rows_accumulate_runs(int dtype, const void* rows, int64_t n_rows, int64_t width, const int32_t* rowptr,
                              const int32_t* target, int64_t n_segments, int32_t run, void* out, int64_t n_out_rows,
                              void* stream) {
  if (run < 1 || run > 1024) return fail("tace_rows_accumulate_runs: run must be 1..1024");
  return rows_accumulate(dtype, rows, n_rows, width, rowptr, nullptr, target, n_segments, run, out, n_out_rows,
                         stream);
}

static int rows_accumulate(int dtype, const void* rows, int64_t n_rows, int64_t width, const int32_t* rowptr,
                           const int32_t* slot, const int32_t* target, int64_t n_segments, int32_t run, void* out,
                           int64_t n_out_rows, void* stream) {
  if (n_rows < 0 || width <= 0 || n_segments < 0 || n_segments > INT32_MAX || n_out_rows < 0)
    return fail("tace_rows_accumulate: bad sizes");
  if (n_segments == 0) return 0;
  if (!rowptr || !out || (n_rows > 0 && !rows)) return fail("tace_rows_accumulate: null pointer");
  if (!target && n_segments > n_out_rows) return fail("tace_rows_accumulate: more segments than output rows");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)n_segments), b(256);
  const int esz = dtype == TACE_F64 ? 8 : 4;
  const bool vec = (width * esz) % 16 == 0 && ((uintptr_t)rows & 15) == 0 && ((uintptr_t)out & 15) == 0;
  if (dtype == TACE_F32) {
    if (vec)
      hipLaunchKernelGGL((k_rows_accumulate<float, 4>), g, b, 0, s, (const float*)rows, width, rowptr, slot, target,
                         (int)n_segments, (float*)out, (int)run);
    else
      hipLaunchKernelGGL((k_rows_accumulate<float, 1>), g, b, 0, s, (const float*)rows, width, rowptr, slot, target,
                         (int)n_segments, (float*)out, (int)run);
  } else if (dtype == TACE_F64) {
    if (vec)
      hipLaunchKernelGGL((k_rows_accumulate<double, 2>), g, b, 0, s, (const double*)rows, width, rowptr, slot, target,
                         (int)n_segments, (double*)out, (int)run);
    else
      hipLaunchKernelGGL((k_rows_accumulate<double, 1>), g, b, 0, s, (const double*)rows, width, rowptr, slot,
                         target, (int)n_segments, (double*)out, (int)run);
  } else {
    return fail("tace_rows_accumulate: dtype must be TACE_F32 or TACE_F64");
  }
  return check_launch("tace_rows_accumulate");
}

int tace_edge_pairs(const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* shifts,
                    int64_t n_nodes, int64_t n_edges, int32_t* work, int32_t* w_rows, int32_t* row_edges,
                    int32_t* row_partner, void* stream) {
  if (n_nodes < 0 || n_edges < 0 || n_nodes > INT32_MAX - 1 || n_edges > INT32_MAX / 4 - 64)
    return fail("tace_edge_pairs: bad sizes");
  if (!rowptr || (n_edges && (!src || !shifts || !work || !w_rows || !row_edges || !row_partner)))
    return fail("tace_edge_pairs: null pointer");
  hipStream_t s = (hipStream_t)stream;
  int* partner = work;
  int* owner = work + n_edges;
  int* rank = work + 2 * n_edges;   // n_edges + 1: rank[n_edges] = number of rows
  int* sums = work + 3 * n_edges + 1;   // block sums of the scan and their scan
  if (n_edges == 0) {
    hipLaunchKernelGGL(k_fill<int>, dim3(1), dim3(256), 0, s, rank, (size_t)1, 0);
    return check_launch("tace_edge_pairs");
  }
  if (n_nodes > 0)
    hipLaunchKernelGGL(k_edge_partner, dim3((unsigned)n_nodes), dim3(64), 0, s, rowptr, eid, src, shifts, partner);
  const unsigned nb = (unsigned)((n_edges + 255) / 256);
  hipLaunchKernelGGL(k_edge_owner, dim3(nb), dim3(256), 0, s, partner, (int)n_edges, owner);
  const int nblk = (int)((n_edges + 1023) / 1024);
  hipLaunchKernelGGL(k_scan_sums, dim3((unsigned)nblk), dim3(256), 0, s, owner, (int)n_edges, sums);
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, s, sums, nblk, sums + nblk);
  hipLaunchKernelGGL(k_scan_apply, dim3((unsigned)nblk), dim3(256), 0, s, owner, (int)n_edges, sums + nblk, rank);
  hipLaunchKernelGGL(k_edge_rows, dim3(nb), dim3(256), 0, s, partner, rank, (int)n_edges, w_rows, row_edges,
                     row_partner);
  return check_launch("tace_edge_pairs");
}

int tace_scan_i32(const int32_t* counts, int64_t n, int32_t* out, void* stream) {
  if (n < 0 || n > INT32_MAX - 1) return fail("tace_scan_i32: bad size");
  if (!counts || !out) return fail("tace_scan_i32: null pointer");
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, (hipStream_t)stream, counts, (int)n, out);
  return check_launch("tace_scan_i32");
}

}  // extern "C"
