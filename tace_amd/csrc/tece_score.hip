// MI355X (gfx950) radial-rotary complex QK score of the TECE attention
// (tace/models/_e3nn/archive/oam_2026_07_05.py:699-754), forward and backward.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/tace_hip.h"
#include "common.h"
#include "tece_common.h"

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
        st_nt<TO>(&erow<L>(gq, e, r, C)[c], G * kv);
        st_nt<TO>(&erow<L>(gk, e, r, C)[c], G * qv);
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
          st_nt<TO>(&erow<L>(gq, e, ir, C)[c], G * (cs * kr - sn * ki));
          st_nt<TO>(&erow<L>(gq, e, ii, C)[c], G * (cs * ki + sn * kr));
          st_nt<TO>(&erow<L>(gk, e, ir, C)[c], G * (cs * qr + sn * qi));
          st_nt<TO>(&erow<L>(gk, e, ii, C)[c], G * (cs * qi - sn * qr));
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


extern "C" {

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

}  // extern "C"
