// MI355X (gfx950) gather + rotation of the node features into the edge frames
// with the radial weighting (tace/models/_e3nn/archive/oam_2026_07_05.py:769-780),
// forward and backward.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"
#include "tece_common.h"

// ----------------------------------------------------- rotate into the frame --
// m[e, r, c] = sum_k W[e, r, k] x[row(e, c), k, c mod C] (k in row r's l block)
// over the 2C channels
// of [x_src | x_dst]: row = rows_src[e] for c < C, rows_dst[e] otherwise
// (the gather, concatenation and wigner bmm of oam_2026_07_05.py:769-771).
// Outputs: ms = m[:, :, :C] and md = m[:, :, C:] (contiguous [E, K, C] each,
// the key / query projection inputs) and, when radial weights w [E, ncomp, 2C]
// are given, mw = w[e, comp(r), c] m[e, r, c] ([E, K, 2C], the radial
// weighting of oam_2026_07_05.py:778-780: +m and -m rows share a component).
// x: [n_rows, K, C] node features in the l layout; rows outside [0, n_rows)
// read as zeros.
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
      for (int d = 0; d < 2 * L + 1; ++d) {   // the columns of row r's block
        const int l = m_l<L>(r);
        if (d > 2 * l) continue;   // constant after unrolling
        a += w[r * K + l * l + d] * xk[l * l + d];
      }
      erow<L>(src ? ms : md, e, r, C)[cc] = out_cvt<TO>(a);
      if (wr) erow<L>(mw, e, r, C2)[c] = out_cvt<TO>(wr[(e * NC + m_comp<L>(r)) * C2 + c] * a);
    }
  }
}

// The same forward for float32 features with VC = 2 or 4 adjacent channels
// per lane (the channel count a multiple of VC): 8- or 16-byte feature and
// radial-weight loads and 4- or 8-byte (bf16) / 8- or 16-byte (float32)
// stores, a half or a quarter of the memory instructions of the kernel above
// (whose sums, over each row's l block in the same order, it gives bit for
// bit).  Needs x and radial_w aligned to VC floats and the output blocks to
// VC elements.  The stores are streamed (non-temporal): the outputs go to the
// GEMMs, L2 is left to the gathered rows.
template <int VC> struct RotinVec;
template <> struct RotinVec<2> { typedef float f __attribute__((ext_vector_type(2))); typedef uint32_t h; };
template <> struct RotinVec<4> {
  typedef float f __attribute__((ext_vector_type(4)));
  typedef uint32_t h __attribute__((ext_vector_type(2)));
};

template <int VC>
__device__ __forceinline__ void st_vec(float* p, const float (&a)[VC]) {
  typename RotinVec<VC>::f v;
#pragma unroll
  for (int i = 0; i < VC; ++i) v[i] = a[i];
  __builtin_nontemporal_store(v, (typename RotinVec<VC>::f*)p);
}
template <int VC>
__device__ __forceinline__ void st_vec(bf16_t* p, const float (&a)[VC]) {
  uint32_t w[VC / 2];
#pragma unroll
  for (int i = 0; i < VC / 2; ++i)
    w[i] = (uint32_t)out_cvt<bf16_t>(a[2 * i]) | ((uint32_t)out_cvt<bf16_t>(a[2 * i + 1]) << 16);
  if constexpr (VC == 2) {
    __builtin_nontemporal_store(w[0], (uint32_t*)p);
  } else {
    typename RotinVec<VC>::h v;
    v[0] = w[0];
    v[1] = w[1];
    __builtin_nontemporal_store(v, (typename RotinVec<VC>::h*)p);
  }
}

template <typename TO, int L, int NP, int VC>
__global__ __launch_bounds__(256) void k_rotin_fwd_vec(const float* __restrict__ x, const float* __restrict__ W,
                                                       const int64_t* __restrict__ rows_src,
                                                       const int64_t* __restrict__ rows_dst,
                                                       const float* __restrict__ wr, int64_t n_rows, int64_t E, int C,
                                                       const Blk<TO> ms, const Blk<TO> md, const Blk<TO> mw) {
  constexpr int K = (L + 1) * (L + 1), NC = (L + 1) * (L + 2) / 2;
  typedef typename RotinVec<VC>::f fv;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const float* w = W + e * K * K;
  const int64_t rs = rows_src[e], rd = rows_dst[e];
  const int C2 = 2 * C;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int c = VC * (lane + 64 * j);
    if (c < C2) {
      const bool src = c < C;
      const int64_t row = src ? rs : rd;
      const int cc = src ? c : c - C;
      const bool ok = row >= 0 && row < n_rows;
      fv xk[K];
#pragma unroll
      for (int kk = 0; kk < K; ++kk) {
        if (ok) {
          xk[kk] = *(const fv*)(x + (row * K + kk) * C + cc);
        } else {
#pragma unroll
          for (int i = 0; i < VC; ++i) xk[kk][i] = 0.f;
        }
      }
#pragma unroll
      for (int r = 0; r < K; ++r) {
        float a[VC];
#pragma unroll
        for (int i = 0; i < VC; ++i) a[i] = 0.f;
#pragma unroll
        for (int d = 0; d < 2 * L + 1; ++d) {   // the columns of row r's block
          const int l = m_l<L>(r);
          if (d > 2 * l) continue;   // constant after unrolling
#pragma unroll
          for (int i = 0; i < VC; ++i) a[i] += w[r * K + l * l + d] * xk[l * l + d][i];
        }
        st_vec<VC>(erow<L>(src ? ms : md, e, r, C) + cc, a);
        if (wr) {
          const fv wv = *(const fv*)(wr + (e * NC + m_comp<L>(r)) * C2 + c);
          float b[VC];
#pragma unroll
          for (int i = 0; i < VC; ++i) b[i] = wv[i] * a[i];
          st_vec<VC>(erow<L>(mw, e, r, C2) + c, b);
        }
      }
    }
  }
}

// backward: with g[e,r,c] = g_ms / g_md [e,r,c mod C] + w[e,comp(r),c] g_mw[e,r,c]
// (absent gradients count as zero):
//   g_x_src[e, k, c] = sum_r W[e,r,k] g[e,r,c] (c < C), g_x_dst the same for
//   channels C..2C-1 (per edge; the caller sums them into the rows);
//   g_W[e, r, k] = sum over the 2C channels of g[e,r,c] x[row(e,c), k, c] on
//   the Wigner matrix's l blocks (row r and column k of one l), zero elsewhere:
//   W is block-diagonal, the forward reads its blocks only, and the entries
//   off them are constants whose gradient nothing uses;
//   g_w[e, comp, c] = sum of g_mw[e,r,c] m[e,r,c] over the rows r of comp.
// Every sum over r or k runs over one l block (the other products are zeros).
// V = 2 (float32, even C, 8-byte aligned operands): two adjacent channels per
// lane, 8-byte loads and stores; g_x and g_w are then the same bits as with
// V = 1, and g_W differs by float rounding (two channels summed per lane
// before the lanes are).
template <typename T, int L, int NS, int V, bool RUNS>
__device__ __forceinline__ void rotin_bwd_edge(const T* __restrict__ x, const T* __restrict__ W,
                                               const int64_t* __restrict__ rows_src,
                                               const int64_t* __restrict__ rows_dst, const T* __restrict__ wr,
                                               const Blk<const T>& gms, const Blk<const T>& gmd,
                                               const Blk<const T>& gmw, int64_t n_rows, int64_t E, int C, int64_t e,
                                               T* __restrict__ gxs, T* __restrict__ gxd, T* __restrict__ gW,
                                               T* __restrict__ gwr, T* __restrict__ lrow, bool accW) {
  constexpr int K = (L + 1) * (L + 1), NB = wig_nb<L>(), P = (NB + 15) / 16 * 16, NC = (L + 1) * (L + 2) / 2;
  const int lane = (int)threadIdx.x & 63;
  const T* w = W + e * K * K;
  const int64_t rs = rows_src[e], rd = rows_dst[e];
  const int C2 = 2 * C;
  T p[P];
#pragma unroll
  for (int i = 0; i < P; ++i) p[i] = T(0);
  // two channels per lane: one slot at a time (its registers not doubled by
  // the next slot's loads)
#pragma unroll(V == 2 ? 1 : NS)
  for (int j = 0; j < NS; ++j) {
    const int c = V * (lane + 64 * j);
    if (c < C2) {
      const bool src = c < C;
      const int64_t row = src ? rs : rd;
      const int cc = src ? c : c - C;
      const bool ok = row >= 0 && row < n_rows;
      const Blk<const T>& gsd = src ? gms : gmd;
      T xk[K][V], g[K][V];
#pragma unroll
      for (int kk = 0; kk < K; ++kk) {
        if (ok) {
          ldv<T, V>(x + (row * K + kk) * C + cc, xk[kk]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) xk[kk][v] = T(0);
        }
      }
#pragma unroll
      for (int r = 0; r < K; ++r) {
        if (gsd.p[mblk<L>(r)]) {
          ldv<T, V>(erow<L>(gsd, e, r, C) + cc, g[r]);
        } else {
#pragma unroll
          for (int v = 0; v < V; ++v) g[r][v] = T(0);
        }
      }
      if (wr) {
        T gc[NC][V];
#pragma unroll
        for (int q = 0; q < NC; ++q)
#pragma unroll
          for (int v = 0; v < V; ++v) gc[q][v] = T(0);
#pragma unroll
        for (int r = 0; r < K; ++r) {
          T gr[V], wv[V];
          if (gmw.p[mblk<L>(r)]) {
            ldv<T, V>(erow<L>(gmw, e, r, C2) + c, gr);
          } else {
#pragma unroll
            for (int v = 0; v < V; ++v) gr[v] = T(0);
          }
          const int q = m_comp<L>(r);
          ldv<T, V>(wr + (e * NC + q) * C2 + c, wv);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            g[r][v] += wv[v] * gr[v];
            T mv = 0;
#pragma unroll
            for (int d = 0; d < 2 * L + 1; ++d) {   // the columns of row r's block
              const int l = m_l<L>(r);
              if (d > 2 * l) continue;   // constant after unrolling
              mv += w[r * K + l * l + d] * xk[l * l + d][v];
            }
            gc[q][v] += gr[v] * mv;
          }
        }
        if (gwr) {
#pragma unroll
          for (int q = 0; q < NC; ++q) stv_nt<T, V>(gwr + (e * NC + q) * C2 + c, gc[q]);
        }
      }
#pragma unroll
      for (int kk = 0; kk < K; ++kk) {
        T a[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          a[v] = T(0);
#pragma unroll
          for (int i = 0; i < 2 * L + 1; ++i) {   // the rows of column kk's block, in order
            const int l = l_of(kk);
            if (i > 2 * l) continue;
            const int r = blk_row<L>(l, i);
            a[v] += w[r * K + kk] * g[r][v];
          }
        }
        if (RUNS && !src)
          stv<T, V>(lrow + kk * C + cc, a);
        else
          stv_nt<T, V>((src ? gxs : gxd) + (e * K + kk) * C + cc, a);
      }
#pragma unroll
      for (int r = 0; r < K; ++r)
#pragma unroll
        for (int d = 0; d < 2 * L + 1; ++d) {
          const int l = m_l<L>(r);
          if (d > 2 * l) continue;
          const int t = wig_row_off<L>(r) + d;
#pragma unroll
          for (int v = 0; v < V; ++v) p[t] += g[r][v] * xk[l * l + d][v];
        }
    }
  }
  // lane sums of the compact entries, then every entry of g_W (zeros off the blocks)
#pragma unroll
  for (int gq = 0; gq < P / 16; ++gq) {
    const T t = reduce16_lanes(p[16 * gq], p[16 * gq + 1], p[16 * gq + 2], p[16 * gq + 3], p[16 * gq + 4],
                               p[16 * gq + 5], p[16 * gq + 6], p[16 * gq + 7], p[16 * gq + 8], p[16 * gq + 9],
                               p[16 * gq + 10], p[16 * gq + 11], p[16 * gq + 12], p[16 * gq + 13], p[16 * gq + 14],
                               p[16 * gq + 15]);
    const int i = 16 * gq + rev4(lane);
    if (lane < 16 && i < NB) {
      int r = 0;
      while (r + 1 < K && wig_row_off<L>(r + 1) <= i) ++r;
      const int l = m_l<L>(r);
      T* dst = gW + e * K * K + r * K + l * l + (i - wig_row_off<L>(r));
      *dst = accW ? *dst + t : t;
    }
  }
  if (accW) return;   // the entries off the blocks hold the caller's zeros
  for (int i = lane; i < K * K; i += 64) {
    const int r = i / K, kk = i - r * K;
    if (l_of(kk) != m_l<L>(r)) gW[e * K * K + i] = T(0);
  }
}

// One edge per wavefront (4 per workgroup).
// RUNS (edges in receiver-CSR order, dynamic LDS of 4 K C values): the four
// edges of a workgroup put their receiver rows in LDS, and each run of edges
// with the same receiver row writes one row, the run's sum in edge order, at
// the run's first position; positions inside a run are left unwritten.  A
// run starts at a receiver's first edge or at a multiple of 4, which is what
// tace_rows_accumulate_runs reads (run = 4).
template <typename T, int L, int NS, int V, bool RUNS>
__global__ __launch_bounds__(256) void k_rotin_bwd(const T* __restrict__ x, const T* __restrict__ W,
                                                   const int64_t* __restrict__ rows_src,
                                                   const int64_t* __restrict__ rows_dst, const T* __restrict__ wr,
                                                   const Blk<const T> gms, const Blk<const T> gmd,
                                                   const Blk<const T> gmw, int64_t n_rows, int64_t E, int C,
                                                   T* __restrict__ gxs, T* __restrict__ gxd, T* __restrict__ gW,
                                                   T* __restrict__ gwr, bool accW) {
  constexpr int K = (L + 1) * (L + 1);
  extern __shared__ __attribute__((aligned(16))) unsigned char rb_raw[];
  const int64_t e = wave_edge();
  if (!RUNS && e >= E) return;
  if (e < E)
    rotin_bwd_edge<T, L, NS, V, RUNS>(x, W, rows_src, rows_dst, wr, gms, gmd, gmw, n_rows, E, C, e, gxs, gxd, gW,
                                      gwr, (T*)rb_raw + (threadIdx.x >> 6) * K * C, accW);
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


extern "C" {

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
  // float32 features: VC = 4 (or 2) channels per lane when the channel count
  // is a multiple of VC, x and radial_w are aligned to VC floats and the
  // outputs to VC elements
  auto aligned = [&](int vc) {
    if (!(dtype == TACE_F32 || dtype == TACE_F32_BF16) || channels % vc || channels > 512) return false;
    const size_t xal = 4 * (size_t)vc, oal = (dtype == TACE_F32_BF16 ? 2 : 4) * (size_t)vc;
    if (((uintptr_t)x % xal) || ((uintptr_t)radial_w % xal)) return false;
    for (int m = 0; m <= lmax; ++m)
      if (((uintptr_t)m_src[m] % oal) || ((uintptr_t)m_dst[m] % oal) || (radial_w && ((uintptr_t)m_w[m] % oal)))
        return false;
    return true;
  };
  const int vc = aligned(4) ? 4 : aligned(2) ? 2 : 1;
  if (vc > 1) {
#define RI_V(TO, LL, VCC)                                                                                     \
  TACE_SLOTS_DISPATCH(2 * channels / (VCC), NP,                                                              \
    hipLaunchKernelGGL((k_rotin_fwd_vec<TO, LL, NP, VCC>), g, b, 0, s, (const float*)x, (const float*)wigner,  \
                       rows_src, rows_dst, (const float*)radial_w, n_rows, n_edges, channels,                  \
                       blocks_of<TO>(m_src, lmax), blocks_of<TO>(m_dst, lmax),                                 \
                       blocks_of<TO>(radial_w ? m_w : nullptr, lmax)))
#define RI_VL(TO, VCC)                                                                                        \
  if (lmax == 1) { RI_V(TO, 1, VCC) } else if (lmax == 2) { RI_V(TO, 2, VCC) } else { RI_V(TO, 3, VCC) }
    if (dtype == TACE_F32) {
      if (vc == 4) { RI_VL(float, 4) } else { RI_VL(float, 2) }
    } else {
      if (vc == 4) { RI_VL(bf16_t, 4) } else { RI_VL(bf16_t, 2) }
    }
#undef RI_VL
#undef RI_V
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

// Two channels per lane for the rotate-in backward: float32, an even channel
// count and every operand 8-byte aligned.
static bool rotin_bwd_pairs(int dtype, int32_t channels, int32_t lmax, const void* x, const void* radial_w,
                            const void* const* g_m_src, const void* const* g_m_dst, const void* const* g_m_w,
                            const void* g_x_src, const void* g_x_dst, const void* g_radial_w) {
  // (lmax 3 would hold 84 W-gradient sums and 2 x 16 x 2 operands per lane:
  // past 256 VGPRs, so it stays on one channel per lane)
  if (dtype != TACE_F32 || (channels & 1) || channels > 512 || lmax > 2) return false;
  auto al = [](const void* q) { return ((uintptr_t)q & 7) == 0; };
  if (!al(x) || !al(radial_w) || !al(g_x_src) || !al(g_x_dst) || !al(g_radial_w)) return false;
  for (int m = 0; m <= lmax; ++m)
    if (!al(g_m_src ? g_m_src[m] : nullptr) || !al(g_m_dst ? g_m_dst[m] : nullptr) ||
        !al(g_m_w ? g_m_w[m] : nullptr))
      return false;
  return true;
}

static int tace_edge_rotate_in_bwd_impl(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                                        const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                                        const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows,
                                        int64_t n_edges, int32_t lmax, int32_t channels, void* g_x_src,
                                        void* g_x_dst, void* g_wigner, void* g_radial_w, bool runs, bool acc_wigner,
                                        void* stream) {
  const char* who = runs ? "tace_edge_rotate_in_bwd_runs" : "tace_edge_rotate_in_bwd";
  if (rotin_checks(who, n_rows, n_edges, lmax, channels)) return -1;
  const size_t es = dtype == TACE_F64 ? 8 : 4;
  const size_t lds = runs ? (size_t)4 * (lmax + 1) * (lmax + 1) * channels * es : 0;
  char msg[160];
  if (lds > 65536) {
    snprintf(msg, sizeof(msg), "%s: 4 (lmax+1)^2 channels values exceed 64 KB of LDS", who);
    return tace_fail_msg(msg);
  }
  if (n_edges == 0) return 0;
  if (!x || !wigner || !rows_src || !rows_dst || !g_x_src || !g_x_dst || !g_wigner || (g_m_w && !radial_w)) {
    snprintf(msg, sizeof(msg), "%s: null pointer", who);
    return tace_fail_msg(msg);
  }
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
  const bool pairs = rotin_bwd_pairs(dtype, channels, lmax, x, radial_w, g_m_src, g_m_dst, g_m_w, g_x_src, g_x_dst,
                                     g_radial_w);
#define RI_B(TT, LL, VV, RR, SLOTS)                                                                             \
  TACE_SLOTS_DISPATCH(SLOTS, NS,                                                                               \
    hipLaunchKernelGGL((k_rotin_bwd<TT, LL, NS, VV, RR>), g, b, lds, s, (const TT*)x, (const TT*)wigner,        \
                       rows_src, rows_dst, (const TT*)radial_w, blocks_of<const TT>(g_m_src, lmax),             \
                       blocks_of<const TT>(g_m_dst, lmax), blocks_of<const TT>(g_m_w, lmax), n_rows, n_edges,    \
                       channels, (TT*)g_x_src, (TT*)g_x_dst, (TT*)g_wigner, (TT*)g_radial_w, acc_wigner))
#define RI_BL(TT, VV, RR, SLOTS)                                                                                  \
  if (lmax == 1) { RI_B(TT, 1, VV, RR, SLOTS) } else if (lmax == 2) { RI_B(TT, 2, VV, RR, SLOTS) }             \
  else { RI_B(TT, 3, VV, RR, SLOTS) }
#define RI_BP(RR)                                                                                             \
  if (channels <= 64) { RI_BP_L(RR, 1) } else if (channels <= 128) { RI_BP_L(RR, 2) }                       \
  else if (channels <= 256) { RI_BP_L(RR, 4) } else { RI_BP_L(RR, 8) }
#define RI_BP_L(RR, NSP)                                                                                      \
  if (lmax == 1) { RI_BP_K(1, RR, NSP) } else { RI_BP_K(2, RR, NSP) }
#define RI_BP_K(LL, RR, NSP)                                                                                  \
  hipLaunchKernelGGL((k_rotin_bwd<float, LL, NSP, 2, RR>), g, b, lds, s, (const float*)x, (const float*)wigner, \
                     rows_src, rows_dst, (const float*)radial_w, blocks_of<const float>(g_m_src, lmax),          \
                     blocks_of<const float>(g_m_dst, lmax), blocks_of<const float>(g_m_w, lmax), n_rows, n_edges,  \
                     channels, (float*)g_x_src, (float*)g_x_dst, (float*)g_wigner, (float*)g_radial_w, acc_wigner);
  if (pairs) {
    // channel pairs: lmax <= 2 and channels <= 512 (rotin_bwd_pairs)
    if (runs) { RI_BP(true) } else { RI_BP(false) }
  } else if (dtype == TACE_F32) {
    if (runs) { RI_BL(float, 1, true, 2 * channels) } else { RI_BL(float, 1, false, 2 * channels) }
  } else if (dtype == TACE_F64) {
    if (runs) { RI_BL(double, 1, true, 2 * channels) } else { RI_BL(double, 1, false, 2 * channels) }
  } else {
    snprintf(msg, sizeof(msg), "%s: dtype must be TACE_F32 or TACE_F64", who);
    return tace_fail_msg(msg);
  }
#undef RI_BP_K
#undef RI_BP_L
#undef RI_BP
#undef RI_BL
#undef RI_B
  return tace_check_launch(who);
}

int tace_edge_rotate_in_bwd(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                            const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                            const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows, int64_t n_edges,
                            int32_t lmax, int32_t channels, void* g_x_src, void* g_x_dst, void* g_wigner,
                            void* g_radial_w, int32_t accumulate_wigner, void* stream) {
  return tace_edge_rotate_in_bwd_impl(dtype, x, wigner, rows_src, rows_dst, radial_w, g_m_src, g_m_dst, g_m_w,
                                      n_rows, n_edges, lmax, channels, g_x_src, g_x_dst, g_wigner, g_radial_w,
                                      false, accumulate_wigner != 0, stream);
}

int tace_edge_rotate_in_bwd_runs(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                                 const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                                 const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows,
                                 int64_t n_edges, int32_t lmax, int32_t channels, void* g_x_src, void* g_x_dst_runs,
                                 void* g_wigner, void* g_radial_w, int32_t accumulate_wigner, void* stream) {
  return tace_edge_rotate_in_bwd_impl(dtype, x, wigner, rows_src, rows_dst, radial_w, g_m_src, g_m_dst, g_m_w,
                                      n_rows, n_edges, lmax, channels, g_x_src, g_x_dst_runs, g_wigner, g_radial_w,
                                      true, accumulate_wigner != 0, stream);
}

}  // extern "C"
