// MI355X (gfx950) attention-weighted inverse rotation and receiver sum of the
// TECE messages (tace/models/_e3nn/archive/oam_2026_07_05.py:799-823), CSR,
// written in the group-major node layout; forward and backward.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"
#include "tece_common.h"

// --------------------------------------------------- rotate out + scatter --
// out[n, k, c] = sum_{e -> n} sum_r W[e, r, k] alpha[e, c / Ch] m[e, r, c]
// (r in column k's l block: the Wigner matrix's blocks only are read)
// written group-major (block l of the output = [NN, 2l+1, C] at NN*C*l^2, NN
// output rows) at feature row map[n].  One workgroup per receiver, one lane
// per channel.
template <typename T, int L>
__global__ __launch_bounds__(512) void k_rotout_fwd(const Blk<const T> m, const T* __restrict__ alpha,
                                                    const T* __restrict__ W, const int* __restrict__ rowptr,
                                                    const int* __restrict__ eid, const int* __restrict__ map,
                                                    int N, int64_t NN, int C, int H, T* __restrict__ out) {
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
      for (int d = 0; d < 2 * L + 1; ++d) {   // row r's l block
        const int l = m_l<L>(r);
        if (d > 2 * l) continue;   // constant after unrolling
        acc[l * l + d] += w[r * K + l * l + d] * v[r];
      }
  }
  const int n = map ? map[n0] : n0;
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
//   g_W[e,r,k] = sum_c alpha[e,h(c)] m[e,r,c] g[n,k,c] on the Wigner matrix's
//   l blocks, zero elsewhere (as in the rotate-in backward: W is
//   block-diagonal and only its blocks are read).
// Sums over k run over row r's l block.  V = 2 (float32, even channels per
// head, 8-byte aligned m, gout and outputs aligned to two elements): two
// adjacent channels per lane, one slot at a time; g_m is then the same bits
// as with V = 1, g_alpha and g_W equal up to float rounding.
__device__ __forceinline__ void st_pair_v(float* p, float a, float b) { *(float2*)p = make_float2(a, b); }
__device__ __forceinline__ void st_pair_v(bf16_t* p, float a, float b) {
  *(uint32_t*)p = (uint32_t)out_cvt<bf16_t>(a) | ((uint32_t)out_cvt<bf16_t>(b) << 16);
}

template <typename T, typename TO, int L, int NS, int V>
__global__ __launch_bounds__(256) void k_rotout_bwd(const Blk<const T> m, const T* __restrict__ alpha,
                                                    const T* __restrict__ W, const T* __restrict__ gout,
                                                    const int64_t* __restrict__ dst, const int* __restrict__ map,
                                                    int N, int64_t E, int C, int H, const Blk<TO> gm,
                                                    T* __restrict__ galpha, T* __restrict__ gW) {
  constexpr int K = (L + 1) * (L + 1), NB = wig_nb<L>(), P = (NB + 15) / 16 * 16;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const int Ch = C / H, ChL = Ch / V;   // channels per head, and lanes per head
  const int64_t n0 = dst[e];
  const bool okn = n0 >= 0 && n0 < N;
  const int64_t n = okn ? (map ? (int64_t)map[n0] : n0) : 0;
  const int64_t NN = N;
  const T* w = W + e * K * K;
  T p[P];
#pragma unroll
  for (int i = 0; i < P; ++i) p[i] = T(0);
  T run[1] = {T(0)};
#pragma unroll(V == 2 ? 1 : NS)
  for (int j = 0; j < NS; ++j) {
    if (64 * j * V >= C) break;
    const int c = V * (lane + 64 * j);
    const bool act = c < C;
    const int h = act ? c / Ch : 0;
    const T a = alpha[e * H + h];
    T g[K][V];
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      const int l = l_of(kk), jj = kk - l * l;
      if (act && okn) {
        ldv<T, V>(gout + NN * C * l * l + (n * (2 * l + 1) + jj) * C + c, g[kk]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) g[kk][v] = T(0);
      }
    }
    T vs[1] = {T(0)};
    if (act) {
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const int l = m_l<L>(r);
        T t[V], mv[V];
        ldv<T, V>(erow<L>(m, e, r, C) + c, mv);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          t[v] = T(0);
#pragma unroll
          for (int d = 0; d < 2 * L + 1; ++d) {   // the columns of row r's block
            if (d > 2 * l) continue;   // constant after unrolling
            t[v] += w[r * K + l * l + d] * g[l * l + d][v];
          }
          vs[0] += mv[v] * t[v];
        }
        if constexpr (V == 2)
          st_pair_v(erow<L>(gm, e, r, C) + c, a * t[0], a * t[1]);
        else
          erow<L>(gm, e, r, C)[c] = out_cvt<TO>(a * t[0]);
#pragma unroll
        for (int d = 0; d < 2 * L + 1; ++d) {
          if (d > 2 * l) continue;
          const int q = wig_row_off<L>(r) + d;
#pragma unroll
          for (int v = 0; v < V; ++v) p[q] += (a * mv[v]) * g[l * l + d][v];
        }
      }
    }
    if (head_sum<T, 1>(vs, run, j, ChL, lane) && act) galpha[e * H + h] = vs[0];
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
      gW[e * K * K + r * K + l * l + (i - wig_row_off<L>(r))] = t;
    }
  }
  for (int i = lane; i < K * K; i += 64) {
    const int r = i / K, kk = i - r * K;
    if (l_of(kk) != m_l<L>(r)) gW[e * K * K + i] = T(0);
  }
}


extern "C" {

static int rotout_checks(const char* who, int64_t N, int32_t lmax, int32_t C, int32_t H) {
  char msg[160];
  if (N < 0 || N > INT32_MAX || lmax < 1 || lmax > 3 || C <= 0 || C > TACE_MAX_CHANNELS || H <= 0 || C % H ||
      (C / H < 64 ? 64 % (C / H) : (C / H) % 64)) {
    snprintf(msg, sizeof(msg), "%s: bad sizes (lmax 1..3, channels <= %d, divisible by heads; per-head width a "
             "divisor or a multiple of 64)", who, TACE_MAX_CHANNELS);
    return tace_fail_msg(msg);
  }
  return 0;
}

int tace_tece_rotate_out_fwd(int dtype, const void* const* m, const void* alpha, const void* wigner,
                             const int32_t* rowptr,
                             const int32_t* eid, const int32_t* node_map, int64_t n_nodes, int64_t out_rows,
                             int32_t lmax, int32_t channels, int32_t heads, void* out, void* stream) {
  if (rotout_checks("tace_tece_rotate_out_fwd", n_nodes, lmax, channels, heads)) return -1;
  if (out_rows == 0) out_rows = n_nodes;
  if (out_rows < 0 || (out_rows != n_nodes && !node_map))
    return tace_fail_msg("tace_tece_rotate_out_fwd: out_rows other than n_nodes needs a node_map");
  if (n_nodes == 0) return 0;
  if (!rowptr || !out) return tace_fail_msg("tace_tece_rotate_out_fwd: null pointer");
  if (!m) return tace_fail_msg("tace_tece_rotate_out_fwd: null block array");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)n_nodes), b((unsigned)((channels + 63) / 64 * 64));
#define ROT_F(TT, LL)                                                                                           \
  hipLaunchKernelGGL((k_rotout_fwd<TT, LL>), g, b, 0, s, blocks_of<const TT>(m, lmax), (const TT*)alpha,      \
                     (const TT*)wigner, rowptr, eid, node_map, (int)n_nodes, out_rows, channels, heads, (TT*)out)
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
    hipLaunchKernelGGL((k_rotout_bwd<TT, TO, LL, NS, 1>), g, b, 0, s, blocks_of<const TT>(m, lmax),          \
                       (const TT*)alpha, (const TT*)wigner, (const TT*)g_out, dst, node_map, (int)n_nodes,    \
                       n_edges, channels, heads, blocks_of<TO>(g_m, lmax), (TT*)g_alpha, (TT*)g_wigner))
  // two channels per lane: float32 features, lmax <= 2, an even channel count
  // per head, up to 512 channels, m and g_out 8-byte aligned and g_m aligned
  // to two elements
  bool pairs = (dtype == TACE_F32 || dtype == TACE_F32_BF16) && lmax <= 2 && ((channels / heads) & 1) == 0 &&
               channels <= 512 && ((uintptr_t)g_out & 7) == 0;
  const size_t gal = dtype == TACE_F32_BF16 ? 4 : 8;
  for (int q = 0; pairs && q <= lmax; ++q)
    pairs = ((uintptr_t)m[q] & 7) == 0 && ((uintptr_t)g_m[q] % gal) == 0;
  if (pairs) {
#define ROT_BP_K(TO, LL, NSP)                                                                                \
  hipLaunchKernelGGL((k_rotout_bwd<float, TO, LL, NSP, 2>), g, b, 0, s, blocks_of<const float>(m, lmax),      \
                     (const float*)alpha, (const float*)wigner, (const float*)g_out, dst, node_map, (int)n_nodes, \
                     n_edges, channels, heads, blocks_of<TO>(g_m, lmax), (float*)g_alpha, (float*)g_wigner);
#define ROT_BP_L(TO, NSP) if (lmax == 1) { ROT_BP_K(TO, 1, NSP) } else { ROT_BP_K(TO, 2, NSP) }
#define ROT_BP(TO)                                                                                             \
  if (channels <= 128) { ROT_BP_L(TO, 1) } else if (channels <= 256) { ROT_BP_L(TO, 2) }                     \
  else { ROT_BP_L(TO, 4) }
    if (dtype == TACE_F32) { ROT_BP(float) } else { ROT_BP(bf16_t) }
#undef ROT_BP
#undef ROT_BP_L
#undef ROT_BP_K
    return tace_check_launch("tace_tece_rotate_out_bwd");
  }
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

}  // extern "C"
