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

// VC = 1, 2 or 4 adjacent channels per lane (float32, the head width a
// multiple of VC, operands aligned to VC elements): 4-, 8- or 16-byte
// requests; the per-channel products and the g_q / g_k outputs are those of
// VC = 1, the head sums add a lane's channels first.
template <int VC> struct ScVec;
template <> struct ScVec<2> { typedef float f __attribute__((ext_vector_type(2))); };
template <> struct ScVec<4> { typedef float f __attribute__((ext_vector_type(4))); };

template <typename T, int VC>
__device__ __forceinline__ void ld_vc(const T* p, T (&o)[VC]) {
  if constexpr (VC == 1) {
    o[0] = *p;
  } else {
    static_assert(sizeof(T) == 4, "several channels per lane: float32 only");
    const typename ScVec<VC>::f v = *(const typename ScVec<VC>::f*)p;
#pragma unroll
    for (int i = 0; i < VC; ++i) o[i] = v[i];
  }
}

template <typename TO, typename T, int VC>
__device__ __forceinline__ void st_vc_nt(TO* p, const T (&a)[VC]) {
  if constexpr (VC == 1) {
    st_nt<TO>(p, a[0]);
  } else if constexpr (sizeof(TO) == 2) {
    uint32_t w[VC / 2];
#pragma unroll
    for (int i = 0; i < VC / 2; ++i)
      w[i] = (uint32_t)out_cvt<bf16_t>(a[2 * i]) | ((uint32_t)out_cvt<bf16_t>(a[2 * i + 1]) << 16);
    if constexpr (VC == 2) {
      __builtin_nontemporal_store(w[0], (uint32_t*)p);
    } else {
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      u2 v;
      v[0] = w[0];
      v[1] = w[1];
      __builtin_nontemporal_store(v, (u2*)p);
    }
  } else {
    typename ScVec<VC>::f v;
#pragma unroll
    for (int i = 0; i < VC; ++i) v[i] = a[i];
    __builtin_nontemporal_store(v, (typename ScVec<VC>::f*)p);
  }
}

template <typename T, int L, int NS, int VC>
__global__ __launch_bounds__(256) void k_score_fwd(const Blk<const T> q, const Blk<const T> k,
                                                   const T* __restrict__ rp, const T* __restrict__ tscale,
                                                   int64_t E, int C, int H, T* __restrict__ score) {
  constexpr int V = 1 + 2 * L;
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const int Ch = C / H, ChL = Ch / VC;
  T run[V];
#pragma unroll
  for (int i = 0; i < V; ++i) run[i] = T(0);
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j * VC >= C) break;
    const int c = VC * (lane + 64 * j);
    T v[V];
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = T(0);
    if (c < C) {
#pragma unroll
      for (int r = 0; r <= L; ++r) {
        T qv[VC], kv[VC];
        ld_vc<T, VC>(erow<L>(q, e, r, C) + c, qv);
        ld_vc<T, VC>(erow<L>(k, e, r, C) + c, kv);
#pragma unroll
        for (int u = 0; u < VC; ++u) v[0] += qv[u] * kv[u];
      }
#pragma unroll
      for (int m = 1; m <= L; ++m) {
        const int re = m_rows_start<L>(m), n = L + 1 - m;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          T qr[VC], qi[VC], kr[VC], ki[VC];
          ld_vc<T, VC>(erow<L>(q, e, re + i, C) + c, qr);
          ld_vc<T, VC>(erow<L>(q, e, re + n + i, C) + c, qi);
          ld_vc<T, VC>(erow<L>(k, e, re + i, C) + c, kr);
          ld_vc<T, VC>(erow<L>(k, e, re + n + i, C) + c, ki);
#pragma unroll
          for (int u = 0; u < VC; ++u) {
            v[2 * m - 1] += qr[u] * kr[u] + qi[u] * ki[u];
            v[2 * m] += qi[u] * kr[u] - qr[u] * ki[u];
          }
        }
      }
    }
    if (head_sum<T, V>(v, run, j, ChL, lane) && c < C) {
      const int h = c / Ch;
      const T phi = T(M_PI) * tanh(rp[e * 2 * H + H + h]);
      T s = v[0];
#pragma unroll
      for (int m = 1; m <= L; ++m) s += cos(T(m) * phi) * v[2 * m - 1] + sin(T(m) * phi) * v[2 * m];
      score[e * H + h] = s * tscale[h] + rp[e * 2 * H + h];
    }
  }
}

template <typename T, typename TO, int L, int NS, int VC>
__global__ __launch_bounds__(256) void k_score_bwd(const Blk<const T> q, const Blk<const T> k,
                                                   const T* __restrict__ rp, const T* __restrict__ tscale,
                                                   const T* __restrict__ gs, int64_t E, int C, int H,
                                                   const Blk<TO> gq, const Blk<TO> gk, T* __restrict__ grp) {
  const int64_t e = wave_edge();
  if (e >= E) return;
  const int lane = (int)threadIdx.x & 63;
  const int Ch = C / H, ChL = Ch / VC;
  T run[1] = {T(0)};
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (64 * j * VC >= C) break;
    const int c = VC * (lane + 64 * j);
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
        T qv[VC], kv[VC], oq[VC], ok[VC];
        ld_vc<T, VC>(erow<L>(q, e, r, C) + c, qv);
        ld_vc<T, VC>(erow<L>(k, e, r, C) + c, kv);
#pragma unroll
        for (int u = 0; u < VC; ++u) {
          oq[u] = G * kv[u];
          ok[u] = G * qv[u];
        }
        st_vc_nt<TO, T, VC>(erow<L>(gq, e, r, C) + c, oq);
        st_vc_nt<TO, T, VC>(erow<L>(gk, e, r, C) + c, ok);
      }
#pragma unroll
      for (int m = 1; m <= L; ++m) {
        const int re = m_rows_start<L>(m), n = L + 1 - m;
        const T cs = cos(T(m) * phi), sn = sin(T(m) * phi);
        T A = 0, B = 0;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          const int ir = re + i, ii = re + n + i;
          T qr[VC], qi[VC], kr[VC], ki[VC], a0[VC], a1[VC], a2[VC], a3[VC];
          ld_vc<T, VC>(erow<L>(q, e, ir, C) + c, qr);
          ld_vc<T, VC>(erow<L>(q, e, ii, C) + c, qi);
          ld_vc<T, VC>(erow<L>(k, e, ir, C) + c, kr);
          ld_vc<T, VC>(erow<L>(k, e, ii, C) + c, ki);
#pragma unroll
          for (int u = 0; u < VC; ++u) {
            A += qr[u] * kr[u] + qi[u] * ki[u];
            B += qi[u] * kr[u] - qr[u] * ki[u];
            a0[u] = G * (cs * kr[u] - sn * ki[u]);
            a1[u] = G * (cs * ki[u] + sn * kr[u]);
            a2[u] = G * (cs * qr[u] + sn * qi[u]);
            a3[u] = G * (cs * qi[u] - sn * qr[u]);
          }
          st_vc_nt<TO, T, VC>(erow<L>(gq, e, ir, C) + c, a0);
          st_vc_nt<TO, T, VC>(erow<L>(gq, e, ii, C) + c, a1);
          st_vc_nt<TO, T, VC>(erow<L>(gk, e, ir, C) + c, a2);
          st_vc_nt<TO, T, VC>(erow<L>(gk, e, ii, C) + c, a3);
        }
        d[0] += T(m) * (cs * B - sn * A);
      }
    }
    if (head_sum<T, 1>(d, run, j, ChL, lane) && act) {
      grp[e * 2 * H + h] = g;
      grp[e * 2 * H + H + h] = G * d[0] * T(M_PI) * (T(1) - th * th);
    }
  }
}


extern "C" {

// Channels per lane of the score kernels: 4 or 2 (float32, the head width a
// multiple of it and, in lanes, a divisor or a multiple of 64; q, k 16- or
// 8-byte aligned; the gradient blocks aligned to as many elements of out_size
// bytes), else 1.
static int score_vc(int dtype, int32_t C, int32_t H, int32_t lmax, const void* const* q, const void* const* k,
                    const void* const* gq, const void* const* gk, int out_size) {
  if (dtype != TACE_F32 && dtype != TACE_F32_BF16) return 1;
  const int Ch = C / H;
  for (int vc = 4; vc >= 2; vc /= 2) {
    if (Ch % vc) continue;
    const int chl = Ch / vc;
    if (chl < 64 ? 64 % chl : chl % 64) continue;
    if (C / vc > 1024) continue;
    bool ok = true;
    for (int m = 0; m <= lmax && ok; ++m) {
      ok = ((uintptr_t)q[m] % (4 * vc)) == 0 && ((uintptr_t)k[m] % (4 * vc)) == 0;
      if (ok && gq) ok = ((uintptr_t)gq[m] % (out_size * vc)) == 0 && ((uintptr_t)gk[m] % (out_size * vc)) == 0;
    }
    if (ok) return vc;
  }
  return 1;
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

int tace_tece_score_fwd(int dtype, const void* const* q, const void* const* k, const void* radial_proj,
                        const void* tscale, int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads,
                        void* score, void* stream) {
  if (score_checks("tace_tece_score_fwd", n_edges, lmax, channels, heads)) return -1;
  if (n_edges == 0) return 0;
  if (!blocks_ok(q, lmax) || !blocks_ok(k, lmax) || !radial_proj || !tscale || !score)
    return tace_fail_msg("tace_tece_score_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g = wave_grid(n_edges), b(256);
  const int vc = score_vc(dtype, channels, heads, lmax, q, k, nullptr, nullptr, 4);
#define SC_F(TT, LL, VCC)                                                                                       \
  TACE_SLOTS_DISPATCH(channels / (VCC), NS,                                                                     \
    hipLaunchKernelGGL((k_score_fwd<TT, LL, NS, VCC>), g, b, 0, s, blocks_of<const TT>(q, lmax),            \
                       blocks_of<const TT>(k, lmax), (const TT*)radial_proj, (const TT*)tscale, n_edges, channels, \
                       heads, (TT*)score))
#define SC_FL(LL) if (vc == 4) { SC_F(float, LL, 4) } else if (vc == 2) { SC_F(float, LL, 2) } else { SC_F(float, LL, 1) }
  if (dtype == TACE_F32) {
    if (lmax == 1) { SC_FL(1) } else if (lmax == 2) { SC_FL(2) } else { SC_FL(3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { SC_F(double, 1, 1) } else if (lmax == 2) { SC_F(double, 2, 1) } else { SC_F(double, 3, 1) }
  } else {
    return tace_fail_msg("tace_tece_score_fwd: dtype must be TACE_F32 or TACE_F64");
  }
#undef SC_FL
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
  const int vc = score_vc(dtype, channels, heads, lmax, q, k, g_q, g_k, dtype == TACE_F32_BF16 ? 2 : 4);
#define SC_B(TT, TO, LL, VCC)                                                                                   \
  TACE_SLOTS_DISPATCH(channels / (VCC), NS,                                                                     \
    hipLaunchKernelGGL((k_score_bwd<TT, TO, LL, NS, VCC>), g, b, 0, s, blocks_of<const TT>(q, lmax),        \
                       blocks_of<const TT>(k, lmax), (const TT*)radial_proj, (const TT*)tscale,              \
                       (const TT*)g_score, n_edges, channels, heads, blocks_of<TO>(g_q, lmax),               \
                       blocks_of<TO>(g_k, lmax), (TT*)g_radial_proj))
#define SC_BL(TO, LL) \
  if (vc == 4) { SC_B(float, TO, LL, 4) } else if (vc == 2) { SC_B(float, TO, LL, 2) } else { SC_B(float, TO, LL, 1) }
  if (dtype == TACE_F32) {
    if (lmax == 1) { SC_BL(float, 1) } else if (lmax == 2) { SC_BL(float, 2) } else { SC_BL(float, 3) }
  } else if (dtype == TACE_F32_BF16) {
    if (lmax == 1) { SC_BL(bf16_t, 1) } else if (lmax == 2) { SC_BL(bf16_t, 2) } else { SC_BL(bf16_t, 3) }
  } else if (dtype == TACE_F64) {
    if (lmax == 1) { SC_B(double, double, 1, 1) } else if (lmax == 2) { SC_B(double, double, 2, 1) }
    else { SC_B(double, double, 3, 1) }
  } else {
    return tace_fail_msg("tace_tece_score_bwd: dtype must be TACE_F32, TACE_F32_BF16 or TACE_F64");
  }
#undef SC_BL
#undef SC_B
  return tace_check_launch("tace_tece_score_bwd");
}

}  // extern "C"
