// MI355X (gfx950) segmented GEMM of the per-species linears
// (e3nnElementLinear, tace/models/linear.py:377-482: one o3.Linear weight per
// chemical element, applied to the nodes of that element).  On species-sorted,
// group-major node features a per-species linear is, per instruction and
// species, one [(rows of that species) x mul_in] @ [mul_in x mul_out] GEMM.
// With tens of species these GEMMs are tiny and one library launch each costs
// more than its arithmetic; this kernel runs ALL of them -- every output
// block, species and instruction of one linear -- in one launch.
//
// Work is described by a host-built table of square output tiles (edge 128:
// the float32 MFMA kernel, edge 64: the FMA kernel, float32 or float64).  A tile
// lies inside one output block and one species' row range, so one weight
// matrix per contributing instruction serves all its rows.  Per tile (8 x
// int64): out_base (element offset of the tile's first row in y), rows (<= edge),
// n (the block's width = row stride), c0 (first column), bias_off (element
// offset into bias, -1 = none), [cb, ce) (its contributions), unused.  Per
// contribution (4 x int64 + one double scale): x_base (element offset of the
// tile's first row in x), k (width of that input block = row stride), w_off
// (element offset of its weight matrix), trans (0: B = W [k, n] row-major;
// 1: B = W^T with W [n, k] row-major -- the input-gradient direction).
// Output: y[tile] = addend[tile] + alpha * (sum_c scale_c x_c[tile rows] @ B_c
// + bias), every element of every tile written once.  addend is optional (null:
// no term) and may be y itself (y += ...): each element is read before it is
// written, by the lane that writes it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tace_hip.h"
#include "bf16x3.h"

int tace_fail_msg(const char* msg);   // tace_hip.hip
int tace_check_launch(const char* what);

namespace {

constexpr int TM = 64, TN = 64, TK = 16, PAD = 4;

// 256 threads = 16 x 16; thread (ty, tx) owns rows ty*4..ty*4+3 and columns
// tx*4..tx*4+3 of the tile.  A and B stage through LDS k-major (As[k][row],
// Bs[k][col]) so the inner product reads one 4-vector of each per k.
template <typename T>
__global__ __launch_bounds__(256) void k_seg_linear(const T* __restrict__ x, T* y, const T* addend,
                                                    const T* __restrict__ w, const T* __restrict__ bias,
                                                    const int64_t* __restrict__ tiles,
                                                    const int64_t* __restrict__ contribs,
                                                    const double* __restrict__ scales, T alpha) {
  __shared__ T As[TK][TM + PAD];
  __shared__ T Bs[TK][TN + PAD];
  const int64_t* td = tiles + 8 * (int64_t)blockIdx.x;
  const int64_t out_base = td[0];
  const int rows = (int)td[1], n = (int)td[2], c0 = (int)td[3];
  const int64_t bias_off = td[4];
  const int cb = (int)td[5], ce = (int)td[6];
  const int t = (int)threadIdx.x, tx = t & 15, ty = t >> 4;
  T acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = T(0);

  for (int c = cb; c < ce; ++c) {
    const int64_t* cd = contribs + 4 * (int64_t)c;
    const T* __restrict__ xa = x + cd[0];
    const int k = (int)cd[1];
    const T* __restrict__ wb = w + cd[2];
    const bool trans = cd[3] != 0;
    const T sc = (T)scales[c];
    for (int k0 = 0; k0 < k; k0 += TK) {
      // A: 64 rows x 16 k, consecutive threads along k (coalesced rows)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int r = (t >> 4) + 16 * p, kk = t & 15;
        As[kk][r] = (r < rows && k0 + kk < k) ? xa[(int64_t)r * k + k0 + kk] : T(0);
      }
      if (!trans) {
        // B[kk][col] = W[k0+kk][c0+col], consecutive threads along the column
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int kk = (t >> 6) + 4 * p, col = t & 63;
          Bs[kk][col] = (k0 + kk < k && c0 + col < n) ? sc * wb[(int64_t)(k0 + kk) * n + c0 + col] : T(0);
        }
      } else {
        // B[kk][col] = W[c0+col][k0+kk], consecutive threads along k
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int col = (t >> 4) + 16 * p, kk = t & 15;
          Bs[kk][col] = (k0 + kk < k && c0 + col < n) ? sc * wb[(int64_t)(c0 + col) * k + k0 + kk] : T(0);
        }
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < TK; ++kk) {
        T a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
      }
      __syncthreads();
    }
  }
  T bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = c0 + tx * 4 + j;
    bv[j] = (bias_off >= 0 && col < n) ? bias[bias_off + col] : T(0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = ty * 4 + i;
    if (r >= rows) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = c0 + tx * 4 + j;
      if (col >= n) continue;
      const int64_t o = out_base + (int64_t)r * n + col;
      y[o] = alpha * (acc[i][j] + bv[j]) + (addend ? addend[o] : T(0));
    }
  }
}

// Global loads of the float32 MFMA path (k_seg_linear_bf16x3 below): every
// load is a 16-byte load, and the next 32-k chunk's loads are issued before
// the current chunk's MFMAs, so memory latency overlaps the matrix work.
typedef float f4 __attribute__((ext_vector_type(4)));

// one 16-byte load of p[0..3], or the first lim (< 4) elements and zeros
__device__ __forceinline__ f4 seg_ld4(const float* p, bool vec, bool any, int lim) {
  if (vec) return *(const f4*)p;
  f4 v = f4{0.f, 0.f, 0.f, 0.f};
  if (any) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < lim) v[e] = p[e];
  }
  return v;
}

// The MFMA kernels start each output's sum from addend / alpha (so that
// alpha (sum + bias) = addend + alpha (products + bias) up to rounding): the
// addend is read into the accumulators before the first MFMA, its loads in
// flight with the tile's first operand loads, instead of a load-add-store
// round trip per output row in the epilogue.  Rows past `rows` and columns
// past `ce` start from zero (they are not stored).
__device__ __forceinline__ f4 addend_init(const float* __restrict__ a, int64_t o, bool rok, int col, int ce,
                                          bool vec, float inv_alpha) {
  f4 v = f4{0.f, 0.f, 0.f, 0.f};
  if (rok) {
    if (vec && col + 4 <= ce) {
      v = *(const f4*)(a + o);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (col + q < ce) v[q] = a[o + q];
    }
  }
  return inv_alpha == 1.f ? v : v * inv_alpha;
}

// R rows x 32 k of a k-contiguous matrix (row stride k, `nrows` valid rows):
// thread t holds rows t/2 + 128 rr (rr < R/128), k k0 + 16 (t&1) .. +15 --
// one base address per row, four 16-byte loads at constant offsets
template <int R>
__device__ __forceinline__ void seg_load_k(const float* __restrict__ base, int k, int k0, int nrows, bool vec, int t,
                                           f4* v) {
  const int kk = k0 + 16 * (t & 1);
#pragma unroll
  for (int rr = 0; rr < R / 128; ++rr) {
    const int r = (t >> 1) + 128 * rr;
    const float* p = base + (int64_t)r * k + kk;
    const bool ok = r < nrows;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int left = k - (kk + 4 * q);
      v[4 * rr + q] = seg_ld4(p + 4 * q, ok && vec && left >= 4, ok && left > 0, left);
    }
  }
}

// float32 as three bfloat16 terms on the bf16 MFMA (v_mfma_f32_16x16x32_bf16,
// 2.3 PFLOP/s against 0.15 for the float32 MFMA): both operands split into
// three bf16 terms, six products per pair (bf16x3.h: the split is exact and
// the sums carry the rounding of a float32 GEMM).
//
// A tile is 128 x 128: 4 waves in a 2 x 2 grid, each owning 4 x 4 blocks of
// 16 x 16.  Tiles are taken XCD-grouped: workgroup b runs tile (b % 8) * per
// + b / 8, so XCD k works through a contiguous stretch of the table (the
// column tiles of one row tile, the row tiles of one species' weight) and
// shares them in its L2.  The split happens once per element at the LDS
// store, into three planes stored k-contiguous (rows of 32 k + 8 pad:
// 80-byte rows, so the 16 rows of a fragment read fall on distinct banks),
// and an MFMA fragment (8 k of one row) is one 16-byte LDS read.  The
// forward's W [k, n] is loaded two k rows per thread and stored transposed as
// (k, k + 1) pairs.
constexpr int SB_K = 32, SB_STR = SB_K + 8;
// rows of 16 k (four f4 of one row, k-contiguous) -> planes p[row][kofs ..]
template <bool SCALED>
__device__ __forceinline__ void sb_store_k16(unsigned short* lds, int plane, int off, const f4* v, float sc) {
  typedef unsigned u4v __attribute__((ext_vector_type(4)));
  u4v o[3][2];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      unsigned h[3];
      const bx3_f2 u = bx3_f2{v[q][2 * e], v[q][2 * e + 1]};
      bx3_split2(SCALED ? bx3_scale2(u, sc) : u, h);
#pragma unroll
      for (int p = 0; p < 3; ++p) o[p][q >> 1][2 * (q & 1) + e] = h[p];
    }
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    *(u4v*)&lds[p * plane + off] = o[p][0];
    *(u4v*)&lds[p * plane + off + 8] = o[p][1];
  }
}

// 32 k rows x 128 columns of W [k, n] from column c0: thread t holds k rows
// k0 + 2 (t/16) and the next, columns 4 (t%16) + 64 q (q < 2) -- v[2 q + r]
// for row 2 (t/16) + r
__device__ __forceinline__ void sb_load_n(const float* __restrict__ wb, int k, int n, int c0, int k0, bool vec, int t,
                                          f4* v) {
  const int cb = c0 + 4 * (t & 15);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int kk = k0 + 2 * (t >> 4) + r;
    const float* p = wb + (int64_t)kk * n + cb;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int left = n - (cb + 64 * q);
      v[2 * q + r] = seg_ld4(p + 64 * q, kk < k && vec && left >= 4, kk < k && left > 0, left);
    }
  }
}

// Lane t writes its four columns 4 (t%16) + e in the order e = (e' + r) & 3,
// r = (t/4) & 3, so that a store instruction (fixed e') spreads the 16 lanes
// of a row group over distinct banks instead of four.
__device__ __forceinline__ void sb_store_n(unsigned short* lds, int plane, int t, const f4* v, float sc) {
  const int kp = 2 * (t >> 4), r = (t >> 2) & 3;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    f4 u0, u1;   // v rotated left by r
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f4 x0 = v[2 * q], x1 = v[2 * q + 1];
      u0[e] = r == 0 ? x0[e] : r == 1 ? x0[(e + 1) & 3] : r == 2 ? x0[(e + 2) & 3] : x0[(e + 3) & 3];
      u1[e] = r == 0 ? x1[e] : r == 1 ? x1[(e + 1) & 3] : r == 2 ? x1[(e + 2) & 3] : x1[(e + 3) & 3];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      unsigned h[3];   // (k, k + 1) of one column
      bx3_split2(bx3_scale2(bx3_f2{u0[e], u1[e]}, sc), h);
      const int col = 4 * (t & 15) + 64 * q + ((e + r) & 3);
#pragma unroll
      for (int p = 0; p < 3; ++p) *(unsigned*)&lds[p * plane + col * SB_STR + kp] = h[p];
    }
  }
}

__global__ __launch_bounds__(256) void k_seg_linear_bf16x3(const float* __restrict__ x, float* y,
                                                           const float* addend, const float* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           const int64_t* __restrict__ tiles,
                                                           const int64_t* __restrict__ contribs,
                                                           const double* __restrict__ scales, float alpha,
                                                           int n_tiles, int per) {
  constexpr int WM = 4, WN = 4, TR = 128, TC = 128, PL = 128 * SB_STR;   // plane size (bf16)
  __shared__ __attribute__((aligned(16))) unsigned short As[3 * PL];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[3 * PL];
  const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (tile >= n_tiles) return;
  const int64_t* td = tiles + 8 * (int64_t)tile;
  const int64_t out_base = td[0];
  const int rows = (int)td[1], n = (int)td[2], c0 = (int)td[3];
  const int64_t bias_off = td[4];
  const int cb = (int)td[5], ce = (int)td[6];
  const int t = (int)threadIdx.x, lane = t & 63, wv = t >> 6;
  const int wr = (wv >> 1) * 16 * WM, wc = (wv & 1) * 16 * WN;
  const int fr = lane & 15, fg = lane >> 4;
  f4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  const int soff = (t >> 1) * SB_STR + 16 * (t & 1);   // this thread's k16 run of a k-contiguous plane

  for (int c = cb; c < ce; ++c) {
    const int64_t* cd = contribs + 4 * (int64_t)c;
    const float* __restrict__ xa = x + cd[0];
    const int k = (int)cd[1];
    const float* __restrict__ wb = w + cd[2];
    const bool trans = cd[3] != 0;
    const float sc = (float)scales[c];
    const bool xvec = ((((uintptr_t)xa) & 15) == 0) && ((k & 3) == 0);
    const bool wvec = ((((uintptr_t)wb) & 15) == 0) && (((trans ? k : n) & 3) == 0) && ((c0 & 3) == 0);
    const float* __restrict__ wt = wb + (int64_t)c0 * k;
    f4 a[4], b[4];
    auto load = [&](int kc, f4* a, f4* b) {
      seg_load_k<TR>(xa, k, kc, rows, xvec, t, a);
      if (trans) seg_load_k<TC>(wt, k, kc, n - c0, wvec, t, b);
      else sb_load_n(wb, k, n, c0, kc, wvec, t, b);
    };
    auto stage = [&](const f4* a, const f4* b) {
      sb_store_k16<false>(As, PL, soff, a, 1.f);
      if (trans) sb_store_k16<true>(Bs, PL, soff, b, sc);
      else sb_store_n(Bs, PL, t, b, sc);
    };
    auto mma = [&]() {
      bx3_bf8 af[3][WM];
#pragma unroll
      for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int i = 0; i < WM; ++i) af[p][i] = *(const bx3_bf8*)&As[p * PL + (wr + 16 * i + fr) * SB_STR + 8 * fg];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        bx3_bf8 bf[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) bf[p] = *(const bx3_bf8*)&Bs[p * PL + (wc + 16 * j + fr) * SB_STR + 8 * fg];
#pragma unroll
        for (int u = 0; u < 6; ++u)   // the six terms a_i b_j, smallest first
#pragma unroll
          for (int i = 0; i < WM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[BX3_TA[u]][i], bf[BX3_TB[u]], acc[i][j], 0, 0, 0);
      }
    };
    load(0, a, b);
    for (int k0 = 0; k0 < k; k0 += SB_K) {
      stage(a, b);
      __syncthreads();
      if (k0 + SB_K < k) load(k0 + SB_K, a, b);   // next chunk in flight during this chunk's MFMAs
      mma();
      __syncthreads();
    }
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = c0 + wc + 16 * j + fr;
    if (col >= n) continue;
    const float bv = bias_off >= 0 ? bias[bias_off + col] : 0.f;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = wr + 16 * i + 4 * fg + q;
        if (r >= rows) continue;
        const int64_t o = out_base + (int64_t)r * n + col;
        y[o] = alpha * (acc[i][j][q] + bv) + (addend ? addend[o] : 0.f);
      }
  }
}

// ---- the same GEMM with the weights split ahead of time ------------------
// The weights of the per-species linears are constants at inference, so their
// three bf16 terms (with the contribution's scale folded in) are made once,
// by k_split_blocks, into three planes laid out the way the LDS tile holds
// them: per weight block, column-major runs of k_pad = ceil8(k) bf16 (zeros
// past k), column c of the block at w_off + c k_pad of each plane.  The GEMM
// then stages B with plain 16-byte copies -- no split, no transposition, no
// scale -- which removes most of the kernel's VALU work and the transposed
// LDS stores.

// 128 columns x 32 k of one contribution's B: thread t stages column t / 2,
// k k0 + 16 (t & 1) .. + 15, of each plane (two 16-byte loads per plane; a
// k_pad run is a multiple of 8, so each load is wholly inside or outside it)
typedef unsigned u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void sbs_load(const unsigned short* __restrict__ wp, int64_t pstride, int kpad, int ncols,
                                         int k0, int t, u4v* v) {
  const int col = t >> 1, kk = k0 + 16 * (t & 1);
  const unsigned short* p = wp + (int64_t)col * kpad + kk;
#pragma unroll
  for (int pl = 0; pl < 3; ++pl)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool ok = col < ncols && kk + 8 * h < kpad;
      v[2 * pl + h] = ok ? *(const u4v*)(p + pl * pstride + 8 * h) : u4v{0u, 0u, 0u, 0u};
    }
}

__device__ __forceinline__ void sbs_store(unsigned short* lds, int plane, int off, const u4v* v) {
#pragma unroll
  for (int pl = 0; pl < 3; ++pl) {
    *(u4v*)&lds[pl * plane + off] = v[2 * pl];
    *(u4v*)&lds[pl * plane + off + 8] = v[2 * pl + 1];
  }
}

__global__ __launch_bounds__(256) void k_seg_linear_bx3s(const float* __restrict__ x, float* y, const float* addend,
                                                         const unsigned short* __restrict__ wsp, int64_t pstride,
                                                         const float* __restrict__ bias,
                                                         const int64_t* __restrict__ tiles,
                                                         const int64_t* __restrict__ contribs, float alpha,
                                                         int n_tiles, int per) {
  constexpr int WM = 4, WN = 4, TR = 128, PL = 128 * SB_STR;   // plane size (bf16)
  __shared__ __attribute__((aligned(16))) unsigned short As[3 * PL];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[3 * PL];
  const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (tile >= n_tiles) return;
  const int64_t* td = tiles + 8 * (int64_t)tile;
  const int64_t out_base = td[0];
  const int rows = (int)td[1], n = (int)td[2], c0 = (int)td[3];
  const int64_t bias_off = td[4];
  const int cb = (int)td[5], ce = (int)td[6];
  const int t = (int)threadIdx.x, lane = t & 63, wv = t >> 6;
  const int wr = (wv >> 1) * 16 * WM, wc = (wv & 1) * 16 * WN;
  const int fr = lane & 15, fg = lane >> 4;
  f4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  const int soff = (t >> 1) * SB_STR + 16 * (t & 1);   // this thread's k16 run of a k-contiguous plane

  for (int c = cb; c < ce; ++c) {
    const int64_t* cd = contribs + 4 * (int64_t)c;
    const float* __restrict__ xa = x + cd[0];
    const int k = (int)cd[1];
    const int kpad = (k + 7) & ~7;
    const unsigned short* __restrict__ wp = wsp + cd[2] + (int64_t)c0 * kpad;
    const bool xvec = ((((uintptr_t)xa) & 15) == 0) && ((k & 3) == 0);
    f4 a[4];
    u4v b[6];
    auto load = [&](int kc) {
      seg_load_k<TR>(xa, k, kc, rows, xvec, t, a);
      sbs_load(wp, pstride, kpad, n - c0, kc, t, b);
    };
    auto mma = [&]() {
      bx3_bf8 af[3][WM];
#pragma unroll
      for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int i = 0; i < WM; ++i) af[p][i] = *(const bx3_bf8*)&As[p * PL + (wr + 16 * i + fr) * SB_STR + 8 * fg];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        bx3_bf8 bf[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) bf[p] = *(const bx3_bf8*)&Bs[p * PL + (wc + 16 * j + fr) * SB_STR + 8 * fg];
#pragma unroll
        for (int u = 0; u < 6; ++u)   // the six terms a_i b_j, smallest first
#pragma unroll
          for (int i = 0; i < WM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[BX3_TA[u]][i], bf[BX3_TB[u]], acc[i][j], 0, 0, 0);
      }
    };
    load(0);
    for (int k0 = 0; k0 < k; k0 += SB_K) {
      sb_store_k16<false>(As, PL, soff, a, 1.f);
      sbs_store(Bs, PL, soff, b);
      __syncthreads();
      if (k0 + SB_K < k) load(k0 + SB_K);   // next chunk in flight during this chunk's MFMAs
      mma();
      __syncthreads();
    }
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int col = c0 + wc + 16 * j + fr;
    if (col >= n) continue;
    const float bv = bias_off >= 0 ? bias[bias_off + col] : 0.f;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = wr + 16 * i + 4 * fg + q;
        if (r >= rows) continue;
        const int64_t o = out_base + (int64_t)r * n + col;
        y[o] = alpha * (acc[i][j][q] + bv) + (addend ? addend[o] : 0.f);
      }
  }
}

// ---- the tile kernel with B in fragment order ----------------------------
// k_seg_linear_bx3s stages A and B through LDS with two barriers per 32-k
// step; LDS traffic (48 KB of plane stores and 96 KB of fragment reads per
// step and workgroup) then takes about as long as the MFMAs.  Here:
//  * B fragments come straight from the weights pre-split in MFMA fragment
//    order (k_split_blocks layout 1, as the task kernel reads them): one
//    coalesced 16-byte load per lane and fragment, one step ahead;
//  * A (128 rows x 32 k) is loaded two steps ahead and split into the three
//    planes in LDS, double buffered: step s + 1's planes are written after
//    step s's MFMAs, and one barrier per step separates them;
//  * every load is unconditional (past the last step it repeats that step):
//    a load under a branch makes the compiler wait for all loads at the
//    join, the prefetches included;
//  * the MFMA runs with the operands swapped (B fragments as the row
//    operand), so a lane holds 4 consecutive columns of one output row, and
//    the stores trade blocks between lanes fr and fr ^ 8 as the task kernel's
//    do (8 whole rows of 32 columns per store).
// Tiles, contributions and the XCD-grouped tile order are those of
// k_seg_linear_bx3s; contribution column 2 is the block's offset in the
// fragment-order weights.  Per output element the products and their order
// are those of k_seg_linear_bx3s (contributions and k steps in order, the six
// terms smallest first, each a sum over the same 32 products), so the two
// kernels give the same bits.
struct FtLoad {   // the contribution and step whose operands load next
  const float* xa;
  const unsigned short* wf;
  int c, s, k, nks, send;   // steps s .. send - 1 of the contribution's nks
  bool xvec;
};

__device__ __forceinline__ void ft_open(FtLoad& L, const float* __restrict__ x, const unsigned short* __restrict__ wfrag,
                                        const int64_t* __restrict__ contribs, int c) {
  const int64_t* cd = contribs + 4 * (int64_t)c;
  L.c = c;
  L.s = 0;
  L.xa = x + cd[0];
  L.k = (int)cd[1];
  L.nks = (L.k + 31) >> 5;
  L.send = L.nks;
  L.wf = wfrag + cd[2];
  L.xvec = ((((uintptr_t)L.xa) & 15) == 0) && ((L.k & 3) == 0);
}

// A (128 rows x 32 k) of step L.s as seg_load_k<128> holds it, but rows past
// nrows repeat the last row (their outputs are not stored).  VEC (every
// contribution 16-byte aligned with k % 4 == 0): four unconditional 16-byte
// loads, a run past k read from the row's start and zeroed -- no branch, so
// the compiler's wait for this step's B (issued before) is exact.
template <bool VEC>
__device__ __forceinline__ void ft_load_a(const FtLoad& L, int nrows, int t, f4* v) {
  const int kk = 32 * L.s + 16 * (t & 1);
  const int r = min(t >> 1, nrows - 1);
  const float* row = L.xa + (int64_t)r * L.k;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int left = L.k - (kk + 4 * q);
    if constexpr (VEC) {
      const f4 u = *(const f4*)(left >= 4 ? row + kk + 4 * q : row);
      v[q] = left >= 4 ? u : f4{0.f, 0.f, 0.f, 0.f};
    } else {
      v[q] = seg_ld4(row + kk + 4 * q, false, left > 0, left);
    }
  }
}

// B fragments (three terms) of column blocks jb0 .. jb0 + 3 (clamped to the
// block's last) at step L.s
__device__ __forceinline__ void ft_load_b(const FtLoad& L, int jb0, int nb16, int lane, u4v (&d)[3][4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int jb = min(jb0 + j, nb16 - 1);
    const unsigned short* p = L.wf + ((int64_t)(jb * L.nks + L.s) * 3) * 512 + 8 * lane;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) d[pl][j] = *(const u4v*)(p + pl * 512);
  }
}

//
// SPLIT (split k, for launches with too few tiles to fill the chip): work
// item vi = tile * splits + sp sums steps [sp nks / splits, (sp + 1) nks /
// splits) of the tile's first contribution into its own 128 x 128 partial
// tile, partials + 16384 vi (row stride 128), with no addend, bias or alpha;
// k_seg_split_sum adds the partials up (NaN for a tile with more than one
// contribution).
template <bool VEC, bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_seg_linear_bx3f(
    const float* __restrict__ x, float* y, const float* addend,
                                                         const unsigned short* __restrict__ wfrag,
                                                         const float* __restrict__ bias,
                                                         const int64_t* __restrict__ tiles,
                                                         const int64_t* __restrict__ contribs, float alpha,
                                                         int n_tiles, int per, int splits,
                                                         float* __restrict__ partials) {
  constexpr int WM = 4, TR = 128, PL = 128 * SB_STR;   // plane size (bf16)
  __shared__ __attribute__((aligned(16))) unsigned short As[2][3 * PL];
  const int vi = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  const int tile = SPLIT ? vi / splits : vi;
  if (tile >= n_tiles) return;
  const int64_t* td = tiles + 8 * (int64_t)tile;
  const int64_t out_base = td[0];
  const int rows = (int)td[1], n = (int)td[2], c0 = (int)td[3];
  const int64_t bias_off = SPLIT ? -1 : td[4];
  const int cb = (int)td[5];
  int ce = (int)td[6];
  if constexpr (SPLIT) ce = min(ce, cb + 1);   // k_seg_split_sum writes NaN for a tile with more
  const int t = (int)threadIdx.x, lane = t & 63, wv = t >> 6;
  const int wr = (wv >> 1) * 16 * WM, wc = (wv & 1) * 64;
  const int fr = lane & 15, fg = lane >> 4;
  const int nb16 = (n + 15) >> 4, jb0 = (c0 + wc) >> 4;
  const int soff = (t >> 1) * SB_STR + 16 * (t & 1);   // this thread's k16 run of a k-contiguous plane

  f4 acc[WM][4];
  if (!SPLIT && addend) {
    const bool avec = ((n & 3) == 0) && ((out_base & 3) == 0) && ((((uintptr_t)addend) & 15) == 0);
    const float ia = 1.f / alpha;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = wr + 16 * i + fr, col = c0 + wc + 16 * j + 4 * fg;
        acc[i][j] = addend_init(addend, out_base + (int64_t)r * n + col, r < rows, col, n, avec, ia);
      }
  } else {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }

  // skip contributions without k steps
  int c = cb;
  FtLoad L;
  while (c < ce) {
    ft_open(L, x, wfrag, contribs, c);
    if constexpr (SPLIT) {
      const int sp = vi - tile * splits;
      L.s = (int)((int64_t)sp * L.nks / splits);
      L.send = (int)((int64_t)(sp + 1) * L.nks / splits);
    }
    if (L.send > L.s) break;
    ++c;
  }
  if (c < ce) {
    // the steps of all contributions, in order.  A loads two steps ahead of
    // the MFMAs (cursor LA; A(j) in register set j & 1), B one step ahead
    // (cursor LB): x streams from HBM, the weights from L2
    FtLoad LA = L, LB = L;
    bool moreA = true, moreB = true;
    // C to the step after the one it names; after the last step C stays
    // there (more = false), so the loads below never need a condition
    auto advance = [&](FtLoad& C, bool& more) {
      if (C.s + 1 < C.send) {
        ++C.s;
        return;
      }
      if constexpr (SPLIT) {   // one contribution
        more = false;
        return;
      }
      for (int cc = C.c + 1; cc < ce; ++cc) {
        FtLoad D;
        ft_open(D, x, wfrag, contribs, cc);
        if (D.send > 0) {
          C = D;
          return;
        }
      }
      more = false;
    };
    f4 a0[4], a1[4];
    u4v b0[3][4], b1[3][4];
    ft_load_a<VEC>(LA, rows, t, a0);
    advance(LA, moreA);
    ft_load_b(LB, jb0, nb16, lane, b0);
    advance(LB, moreB);
    ft_load_a<VEC>(LA, rows, t, a1);   // (a repeat of the last step when there is no next)
    advance(LA, moreA);
    sb_store_k16<false>(As[0], PL, soff, a0, 1.f);
    __syncthreads();
    // step g: MFMAs on LDS buffer `buf` (= g & 1) and fragments cur while A(g
    // + 2) loads into al and B(g + 1) into nxt; then A(g + 1) (in as) split
    // into the other buffer
    auto step = [&](int buf, const u4v (&cur)[3][4], u4v (&nxt)[3][4], f4 (&al)[4], const f4 (&as)[4]) {
      const bool have = moreB;
      // B before A: vector loads complete in issue order, so waiting for
      // this step's B (issued last step) does not wait for the A issued
      // after it.  Unconditional (repeats past the last step): a load under
      // a branch makes the compiler wait for every load at the join
      ft_load_b(LB, jb0, nb16, lane, nxt);
      advance(LB, moreB);
      ft_load_a<VEC>(LA, rows, t, al);
      advance(LA, moreA);
      __builtin_amdgcn_sched_barrier(0);
      const unsigned short* Ab = As[buf];
#pragma unroll
      for (int ip = 0; ip < WM / 2; ++ip) {
        bx3_bf8 af[2][3];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int pl = 0; pl < 3; ++pl)
            af[ii][pl] = *(const bx3_bf8*)&Ab[pl * PL + (wr + 32 * ip + 16 * ii + fr) * SB_STR + 8 * fg];
#pragma unroll
        for (int u = 0; u < 6; ++u)   // the six terms a_i b_j, smallest first
#pragma unroll
          for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[2 * ip + ii][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bx3_bf8, cur[BX3_TB[u]][j]), af[ii][BX3_TA[u]], acc[2 * ip + ii][j], 0, 0, 0);
      }
      // the next A's split after the MFMAs (interleaving it measured slower)
      __builtin_amdgcn_sched_barrier(0);
      sb_store_k16<false>(As[buf ^ 1], PL, soff, as, 1.f);
      __syncthreads();
      return have;
    };
    while (step(0, b0, b1, a0, a1) && step(1, b1, b0, a1, a0)) {
    }
  }

  // the bias of this lane's 16 columns (no loads are outstanding here)
  f4 bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bv[j] = f4{0.f, 0.f, 0.f, 0.f};
    if (bias_off >= 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[j][q] = bias[bias_off + min(c0 + wc + 16 * j + 4 * fg + q, n - 1)];
    }
  }
  // acc[i][j][q] = out[row wr + 16 i + fr][column c0 + wc + 16 j + 4 fg + q];
  // per pair of blocks (2 jp, 2 jp + 1) lanes fr and fr ^ 8 trade one block,
  // so a store writes 8 whole rows of 32 columns
  const bool vst = SPLIT || (((n & 3) == 0) && ((out_base & 3) == 0) && ((((uintptr_t)y) & 15) == 0));
  const float osc = SPLIT ? 1.f : alpha;
  const bool lo = fr < 8;
  const int jl = lo ? 0 : 1;
#pragma unroll
  for (int jp = 0; jp < 2; ++jp) {
    const int col = c0 + wc + 32 * jp + 16 * jl + 4 * fg;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const f4 v0 = osc * (acc[i][2 * jp] + bv[2 * jp]), v1 = osc * (acc[i][2 * jp + 1] + bv[2 * jp + 1]);
      const f4 give = lo ? v1 : v0;
      f4 got;
#pragma unroll
      for (int q = 0; q < 4; ++q) got[q] = __shfl_xor(give[q], 8);
      const f4 s0 = lo ? v0 : got, s1 = lo ? got : v1;   // rows 16 i + (fr & 7), + 8
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = wr + 16 * i + 8 * h + (fr & 7);
        if (r >= rows || col >= n) continue;
        const f4 v = h ? s1 : s0;
        float* dst = SPLIT ? partials + 16384 * (int64_t)vi + 128 * r + (col - c0) : y + out_base + (int64_t)r * n + col;
        if (vst) {
          *(f4*)dst = v;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (col + q < n) dst[q] = v[q];
        }
      }
    }
  }
}

// The partial tiles of k_seg_linear_bx3f<*, true> added up, 16 workgroups
// per tile (8 rows each, a thread per 4 columns of a row): y = alpha
// (addend / alpha + partial_0 + ... + partial_{splits-1} + bias), the partials
// in split order (a fixed order, so every run gives the same bits); NaN in
// every output of a tile with more than one contribution (the split kernel
// sums only its first).  The addend may be y itself: each element is read
// and then written by the same thread.
__global__ __launch_bounds__(256) void k_seg_split_sum(float* y, const float* addend, const float* __restrict__ bias,
                                                       const int64_t* __restrict__ tiles,
                                                       const float* __restrict__ partials, int splits, float alpha) {
  const int tile = (int)(blockIdx.x >> 4);
  const int64_t* td = tiles + 8 * (int64_t)tile;
  const int64_t out_base = td[0], bias_off = td[4];
  const int rows = (int)td[1], n = (int)td[2], c0 = (int)td[3];
  const int r = 8 * (int)(blockIdx.x & 15) + ((int)threadIdx.x >> 5), cc = 4 * ((int)threadIdx.x & 31), col = c0 + cc;
  if (r >= rows || col >= n) return;
  const bool bad = td[6] - td[5] > 1;
  const bool vec = ((n & 3) == 0) && ((out_base & 3) == 0) && ((((uintptr_t)y) & 15) == 0);
  const bool avec = vec && ((((uintptr_t)addend) & 15) == 0);
  const int64_t o = out_base + (int64_t)r * n + col;
  f4 acc = addend ? addend_init(addend, o, true, col, n, avec, 1.f / alpha) : f4{0.f, 0.f, 0.f, 0.f};
  const float* __restrict__ P = partials + (int64_t)tile * splits * 16384 + 128 * r + cc;
#pragma unroll 4
  for (int s = 0; s < splits; ++s) acc += *(const f4*)(P + (int64_t)s * 16384);
  f4 b = f4{0.f, 0.f, 0.f, 0.f};
  if (bias_off >= 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (col + q < n) b[q] = bias[bias_off + col + q];
  }
  const f4 out = bad ? f4{NAN, NAN, NAN, NAN} : alpha * (acc + b);
  if (vec && col + 4 <= n) {
    *(f4*)(y + o) = out;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (col + q < n) y[o + q] = out[q];
  }
}

// ---- short k, wide n: the input-gradient shape ---------------------------
// The input gradients of the product-basis contractions are [rows, k = 128]
// x [128, n] with n up to ~5,400 columns per output block.  A 128 x 128 tile
// of the kernel above does four 32-k steps after staging A and B through LDS
// with two barriers per step, then writes its outputs one float per lane.
// Here a workgroup owns one R-row tile of one contribution with k <= KM (R =
// 128 for k <= 128, R = 64 for k <= 256) and a range of columns:
//  * A is split once into the three bf16 planes in LDS (k-contiguous rows of
//    128 + 8 bf16: 272-byte rows, so the 16 rows of a fragment read fall on
//    distinct banks); one barrier, none after it;
//  * KS_GROUPS groups of four wavefronts take the range's 128-column tiles in
//    turn; a wavefront owns all R rows of 32 columns, so each B fragment
//    is loaded by one wavefront only;
//  * B comes from weights pre-split in MFMA fragment order (k_split_blocks,
//    layout 1): the three terms of one 16-column x 32-k fragment are three
//    contiguous 1 KB runs in lane order, so a fragment is one fully
//    coalesced 16-byte load per lane.  Loaded one 32-k step ahead, and across
//    the end of a column tile: the next tile's first step is in flight before
//    this tile's stores, so no wait covers them.  The loads are unconditional
//    (the column block clamped into the weight block);
//  * the MFMA runs with the operands swapped (B fragments as the row operand),
//    so a lane holds 4 consecutive columns of one output row: one 16-byte
//    store per 16 x 16 block.
// The number of 32-k steps is a template parameter (1..KM / 32).  Per output element
// the products and their order are those of k_seg_linear_bx3s (k steps in
// order, the six terms smallest first, each a sum over the same 32 products),
// so the two kernels give the same bits.
//
// Task table (10 x int64): out_base (element offset of the tile's row 0,
// column 0 in y), rows (<= R), n (block width = row stride of y), [cb, ce)
// (the columns, ce <= n), bias_off (-1 none), x_base (element offset of the
// tile's row 0 in x), k (0..KM, the row stride of x; 0 = no contribution:
// the tile is alpha * bias or zero), w_off (the block's offset in the
// fragment-order weights), unused.
// Two instantiations: R = 128 rows per task for k <= 128, R = 64 for k <= 256
// (the A planes take 3 R (KM + 8) bf16 of LDS, ~100 KB either way).  Groups of
// four wavefronts per workgroup and the column stride between one group's
// consecutive tiles:
constexpr int KS_GROUPS = 2, KS_THREADS = 256 * KS_GROUPS, KS_CSTEP = 128 * KS_GROUPS;
template <int R, int KM>
struct KsShape {
  static constexpr int RB = R / 16, STR = KM + 8, PL = R * STR;
};

struct KsTask {
  int64_t out_base, bias_off;
  int rows, n, cb, ce, nks, nb16;
  const unsigned short* wf;
  const float* addend;   // added to the outputs (null: none; may be y)
};

// B fragments (three terms, column blocks 2 wq and 2 wq + 1 of column tile c)
// of step ks into d; the column block clamped to the weight block's last
__device__ __forceinline__ void ks_load_b(const KsTask& T, int c, int ks, int wq, int lane, u4v (&d)[3][2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int jb = min((c >> 4) + 2 * wq + j, T.nb16 - 1);
    const unsigned short* p = T.wf + ((int64_t)(jb * T.nks + ks) * 3) * 512 + 8 * lane;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) d[pl][j] = *(const u4v*)(p + pl * 512);
  }
}

// step KS of a column tile: MFMAs on cur while the next step's fragments
// (or the next tile's first) load into nxt
template <int R, int KM, int NKS, int KS>
__device__ __forceinline__ void ks_step(const unsigned short* __restrict__ As, const KsTask& T, int c, int wq,
                                        int lane, int fr, int fg, f4 (&acc)[R / 16][2], const u4v (&cur)[3][2],
                                        u4v (&nxt)[3][2]) {
  if (KS + 1 < NKS) ks_load_b(T, c, KS + 1, wq, lane, nxt);
  else ks_load_b(T, c + KS_CSTEP, 0, wq, lane, nxt);
  // the loads go out before this step's MFMAs (the scheduler would sink them
  // to the end of the step, where nothing hides their latency)
  __builtin_amdgcn_sched_barrier(0);
  typedef KsShape<R, KM> S;
#pragma unroll
  for (int ip = 0; ip < S::RB / 2; ++ip) {   // row blocks in pairs: four independent accumulators per term
    bx3_bf8 af[2][3];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        af[ii][pl] = *(const bx3_bf8*)&As[pl * S::PL + (32 * ip + 16 * ii + fr) * S::STR + 32 * KS + 8 * fg];
#pragma unroll
    for (int u = 0; u < 6; ++u)   // the six terms a_i b_j, smallest first
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[2 * ip + ii][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bx3_bf8, cur[BX3_TB[u]][j]), af[ii][BX3_TA[u]], acc[2 * ip + ii][j], 0, 0, 0);
  }
  // keep the next step's LDS reads out of this one
  __builtin_amdgcn_sched_barrier(0);
}

// steps KS.. of a column tile; step KS reads buffer (KS + PAR) & 1
template <int R, int KM, int NKS, int PAR, int KS>
__device__ __forceinline__ void ks_steps(const unsigned short* __restrict__ As, const KsTask& T, int c, int wq,
                                         int lane, int fr, int fg, f4 (&acc)[R / 16][2], u4v (&b0)[3][2],
                                         u4v (&b1)[3][2]) {
  if constexpr (KS < NKS) {
    if constexpr (((KS + PAR) & 1) == 0) ks_step<R, KM, NKS, KS>(As, T, c, wq, lane, fr, fg, acc, b0, b1);
    else ks_step<R, KM, NKS, KS>(As, T, c, wq, lane, fr, fg, acc, b1, b0);
    ks_steps<R, KM, NKS, PAR, KS + 1>(As, T, c, wq, lane, fr, fg, acc, b0, b1);
  }
}

// this wavefront's 128 x 32 part of column tile c
template <int R, int KM, int NKS, int PAR>
__device__ __forceinline__ void ks_tile(const unsigned short* __restrict__ As, const KsTask& T, float* y,
                                        const float* __restrict__ bias, float alpha, bool vst, int c, int wq,
                                        int lane, int fr, int fg, u4v (&b0)[3][2], u4v (&b1)[3][2]) {
  // the bias of this lane's 8 columns, loaded before the MFMAs: a load
  // waited for in the stores would wait for the B fragments loaded after it
  f4 bv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) bv[j] = f4{0.f, 0.f, 0.f, 0.f};
  if (T.bias_off >= 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[j][q] = bias[T.bias_off + min(c + 32 * wq + 16 * j + 4 * fg + q, T.ce - 1)];
  }
  constexpr int RB = R / 16;
  f4 acc[RB][2];
  if (T.addend) {
    const bool avec = ((T.n & 3) == 0) && ((T.out_base & 3) == 0) && ((((uintptr_t)T.addend) & 15) == 0);
    const float ia = 1.f / alpha;
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = 16 * i + fr, col = c + 32 * wq + 16 * j + 4 * fg;
        acc[i][j] = addend_init(T.addend, T.out_base + (int64_t)r * T.n + col, r < T.rows, col, T.ce, avec, ia);
      }
  } else {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  }
  ks_steps<R, KM, NKS, PAR, 0>(As, T, c, wq, lane, fr, fg, acc, b0, b1);
  // acc[i][j][q] = out[row 16 i + fr][column c + 32 wq + 16 j + 4 fg + q].
  // Lanes fr and fr ^ 8 trade one block, so that a store writes 8 whole rows
  // of the 32 columns (128 contiguous bytes each) instead of 16 half rows:
  // lane fr < 8 keeps j = 0 of row fr and takes j = 0 of row fr + 8; lane
  // fr >= 8 keeps j = 1 of row fr and takes j = 1 of row fr - 8.
  const bool lo = fr < 8;
  const int jl = lo ? 0 : 1;   // this lane's 16-column half, in both stores
  const int col = c + 32 * wq + 16 * jl + 4 * fg;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const f4 v0 = alpha * (acc[i][0] + bv[0]), v1 = alpha * (acc[i][1] + bv[1]);
    const f4 give = lo ? v1 : v0;
    f4 got;
#pragma unroll
    for (int q = 0; q < 4; ++q) got[q] = __shfl_xor(give[q], 8);
    const f4 s0 = lo ? v0 : got, s1 = lo ? got : v1;   // rows 16 i + (fr & 7), + 8
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 16 * i + 8 * h + (fr & 7);
      if (r >= T.rows || col >= T.ce) continue;
      const f4 v = h ? s1 : s0;
      float* dst = y + T.out_base + (int64_t)r * T.n + col;
      if (vst) {
        *(f4*)dst = v;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (col + q < T.ce) dst[q] = v[q];
      }
    }
  }
}

template <int R, int KM, int NKS>
__device__ __forceinline__ void ks_columns(const unsigned short* __restrict__ As, const KsTask& T,
                                           float* y, const float* __restrict__ bias, float alpha, int grp,
                                           int wq, int lane, int fr, int fg) {
  int c0 = T.cb + 128 * grp;
  if (c0 >= T.ce) return;
  // 16-byte stores when every 4-column group of every row is 16-byte aligned
  // (ce and cb are then multiples of 4 too)
  const bool vst = ((T.n & 3) == 0) && ((T.out_base & 3) == 0) && ((((uintptr_t)y) & 15) == 0);
  u4v b0[3][2], b1[3][2];
  if (NKS > 0) ks_load_b(T, c0, 0, wq, lane, b0);
  for (; c0 < T.ce; c0 += 2 * KS_CSTEP) {
    ks_tile<R, KM, NKS, 0>(As, T, y, bias, alpha, vst, c0, wq, lane, fr, fg, b0, b1);
    if (c0 + KS_CSTEP < T.ce)
      ks_tile<R, KM, NKS, NKS & 1>(As, T, y, bias, alpha, vst, c0 + KS_CSTEP, wq, lane, fr, fg, b0, b1);
  }
}

template <int R, int KM>
__global__ __launch_bounds__(KS_THREADS) void k_seg_linear_ks(const float* __restrict__ x, float* y,
                                                       const float* addend,
                                                       const unsigned short* __restrict__ wfrag,
                                                       const float* __restrict__ bias,
                                                       const int64_t* __restrict__ tasks, float alpha, int n_tasks,
                                                       int per) {
  typedef KsShape<R, KM> S;
  __shared__ __attribute__((aligned(16))) unsigned short As[3 * S::PL];
  const int task = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (task >= n_tasks) return;
  const int64_t* td = tasks + 10 * (int64_t)task;
  KsTask T;
  T.out_base = td[0];
  T.rows = (int)td[1];
  T.n = (int)td[2];
  T.cb = (int)td[3];
  T.ce = (int)td[4];
  T.bias_off = td[5];
  const int64_t x_base = td[6];
  const int k = (int)td[7];
  T.wf = wfrag + td[8];
  T.addend = addend;
  T.nks = (k + 31) >> 5;
  T.nb16 = (T.n + 15) >> 4;
  const int t = (int)threadIdx.x, lane = t & 63, wv = t >> 6;
  const int grp = wv >> 2, wq = wv & 3;
  const int fr = lane & 15, fg = lane >> 4;
  if (k < 0 || k > KM) {
    // outside this instantiation's k range: NaN outputs instead of a product
    // of a truncated A tile (the host table builder never makes such tasks)
    for (int u = t; u < T.rows * (T.ce - T.cb); u += KS_THREADS) {
      const int r = u / (T.ce - T.cb), c = T.cb + (u - r * (T.ce - T.cb));
      y[T.out_base + (int64_t)r * T.n + c] = __builtin_nanf("");
    }
    return;
  }

  // A: rows x k of x (row stride k) -> planes, zeros past rows and past k
  // (up to the next multiple of 32)
  {
    const float* __restrict__ xa = x + x_base;
    const bool xvec = ((((uintptr_t)xa) & 15) == 0) && ((k & 3) == 0);
    const int kq = T.nks * 4;   // 8-k units per row
    for (int u = t; u < R * kq; u += KS_THREADS) {
      const int r = u / kq, kk = (u - r * kq) * 8;
      const bool ok = r < T.rows;
      const float* p = xa + (int64_t)r * k + kk;
      const f4 a0 = seg_ld4(p, ok && xvec && kk + 4 <= k, ok && kk < k, k - kk);
      const f4 a1 = seg_ld4(p + 4, ok && xvec && kk + 8 <= k, ok && kk + 4 < k, k - kk - 4);
      const float v[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      bx3_bf8 tt[3];
      bx3_split8(v, tt);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl) *(bx3_bf8*)&As[pl * S::PL + r * S::STR + kk] = tt[pl];
    }
  }
  __syncthreads();

#define KS_C(n) ks_columns<R, KM, (n) <= KM / 32 ? (n) : 0>(As, T, y, bias, alpha, grp, wq, lane, fr, fg)
  switch (T.nks) {
    case 1: KS_C(1); break;
    case 2: KS_C(2); break;
    case 3: KS_C(3); break;
    case 4: KS_C(4); break;
    case 5: KS_C(5); break;
    case 6: KS_C(6); break;
    case 7: KS_C(7); break;
    case 8: KS_C(8); break;
    default: ks_columns<R, KM, 0>(As, T, y, bias, alpha, grp, wq, lane, fr, fg); break;   // k = 0: bias or zeros
  }
#undef KS_C
}

// Per block (6 x int64): src_off, cols, k, transpose, dst_off, layout; one
// double scale.  B[kk][c] = scale * (transpose ? w[src_off + kk cols + c] :
// w[src_off + c k + kk]), zero past k (and past cols).
//  layout 0: column c, k index kk < k_pad = ceil8(k) of term p at
//            out[p * pstride + dst_off + c k_pad + kk];
//  layout 1: MFMA fragment order for k_seg_linear_ks, one buffer: per
//            16-column block cb and 32-k step s (nks = ceil(k / 32) steps),
//            the three terms as 512-element runs in lane order, element
//            (c, kk) of term p at out[dst_off + ((cb nks + s) 3 + p) 512 +
//            (((kk % 32) / 8) 16 + c % 16) 8 + kk % 8], cb = c / 16, s = kk /
//            32, over ceil16(cols) columns.
// blockIdx.y picks the block, the x dimension strides over its elements.
__global__ __launch_bounds__(256) void k_split_blocks(const float* __restrict__ w, const int64_t* __restrict__ blocks,
                                                      const double* __restrict__ scales,
                                                      unsigned short* __restrict__ out, int64_t pstride) {
  const int64_t* bd = blocks + 6 * (int64_t)blockIdx.y;
  const int64_t src = bd[0], dst = bd[4];
  const int cols = (int)bd[1], k = (int)bd[2];
  const bool tr = bd[3] != 0;
  const bool frag = bd[5] == 1;
  const int kpad = frag ? (k + 31) & ~31 : (k + 7) & ~7;
  const int ccols = frag ? (cols + 15) & ~15 : cols;
  const float sc = (float)scales[blockIdx.y];
  const int64_t total = (int64_t)ccols * kpad;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e / kpad), kk = (int)(e - (int64_t)c * kpad);
    float v = 0.f;
    if (kk < k && c < cols)
      v = bx3_scale2(bx3_f2{tr ? w[src + (int64_t)kk * cols + c] : w[src + (int64_t)c * k + kk], 0.f}, sc).x;
    unsigned h[3];
    bx3_split2(bx3_f2{v, 0.f}, h);
    if (frag) {
      const int64_t run = ((int64_t)(c >> 4) * (kpad >> 5) + (kk >> 5)) * 3;
      const int64_t lane_el = (int64_t)((((kk & 31) >> 3) << 4) + (c & 15)) * 8 + (kk & 7);
#pragma unroll
      for (int p = 0; p < 3; ++p) out[dst + (run + p) * 512 + lane_el] = (unsigned short)(h[p] & 0xffffu);
    } else {
#pragma unroll
      for (int p = 0; p < 3; ++p) out[p * pstride + dst + e] = (unsigned short)(h[p] & 0xffffu);
    }
  }
}

}  // namespace

extern "C" int tace_bf16x3_split_blocks(const float* w, const int64_t* blocks, const double* scales,
                                        int64_t n_blocks, uint16_t* planes, int64_t plane_stride, void* stream) {
  if (n_blocks < 0 || n_blocks > 65535) return tace_fail_msg("tace_bf16x3_split_blocks: 0..65535 blocks");
  if (n_blocks == 0) return 0;
  if (!w || !blocks || !scales || !planes) return tace_fail_msg("tace_bf16x3_split_blocks: null pointer");
  if (plane_stride < 0) return tace_fail_msg("tace_bf16x3_split_blocks: bad plane stride");
  hipLaunchKernelGGL(k_split_blocks, dim3(64, (unsigned)n_blocks), dim3(256), 0, (hipStream_t)stream, w, blocks,
                     scales, (unsigned short*)planes, plane_stride);
  return tace_check_launch("tace_bf16x3_split_blocks");
}

extern "C" int tace_seg_linear_presplit(const float* x, float* y, const float* addend, const uint16_t* w_planes,
                                        int64_t plane_stride, const float* bias, const int64_t* tiles,
                                        int64_t n_tiles, const int64_t* contribs, double alpha, void* stream) {
  if (n_tiles < 0 || n_tiles > 0x7ffffff0) return tace_fail_msg("tace_seg_linear_presplit: bad tile count");
  if (n_tiles == 0) return 0;
  if (!x || !y || !w_planes || !tiles || !contribs) return tace_fail_msg("tace_seg_linear_presplit: null pointer");
  if ((((uintptr_t)w_planes) & 15) != 0 || (plane_stride & 7) != 0)
    return tace_fail_msg("tace_seg_linear_presplit: planes must be 16-byte aligned with a stride that is a multiple of 8");
  const int per = (int)((n_tiles + 7) / 8);
  hipLaunchKernelGGL(k_seg_linear_bx3s, dim3((unsigned)(8 * per)), dim3(256), 0, (hipStream_t)stream, x, y,
                     addend, (const unsigned short*)w_planes, plane_stride, bias, tiles, contribs, (float)alpha,
                     (int)n_tiles, per);
  return tace_check_launch("tace_seg_linear_presplit");
}

extern "C" int tace_seg_linear_presplit_frag(const float* x, float* y, const float* addend, const uint16_t* w_frag,
                                             const float* bias,
                                             const int64_t* tiles, int64_t n_tiles, const int64_t* contribs,
                                             int32_t aligned, double alpha, void* stream) {
  if (n_tiles < 0 || n_tiles > 0x7ffffff0) return tace_fail_msg("tace_seg_linear_presplit_frag: bad tile count");
  if (n_tiles == 0) return 0;
  if (!x || !y || !w_frag || !tiles || !contribs) return tace_fail_msg("tace_seg_linear_presplit_frag: null pointer");
  if (addend && alpha == 0.0) return tace_fail_msg("tace_seg_linear_presplit_frag: an addend needs alpha != 0");
  if ((((uintptr_t)w_frag) & 15) != 0)
    return tace_fail_msg("tace_seg_linear_presplit_frag: fragment-order weights must be 16-byte aligned");
  const int per = (int)((n_tiles + 7) / 8);
  const dim3 g((unsigned)(8 * per)), b(256);
  if (aligned && (((uintptr_t)x) & 15) == 0)
    hipLaunchKernelGGL((k_seg_linear_bx3f<true, false>), g, b, 0, (hipStream_t)stream, x, y, addend,
                       (const unsigned short*)w_frag,
                       bias, tiles, contribs, (float)alpha, (int)n_tiles, per, 1, nullptr);
  else
    hipLaunchKernelGGL((k_seg_linear_bx3f<false, false>), g, b, 0, (hipStream_t)stream, x, y, addend,
                       (const unsigned short*)w_frag,
                       bias, tiles, contribs, (float)alpha, (int)n_tiles, per, 1, nullptr);
  return tace_check_launch("tace_seg_linear_presplit_frag");
}

extern "C" int tace_seg_linear_presplit_frag_split(const float* x, float* y, const float* addend,
                                                   const uint16_t* w_frag, const float* bias, const int64_t* tiles,
                                                   int64_t n_tiles, const int64_t* contribs, int32_t aligned,
                                                   int32_t splits, float* partials, int64_t partial_elems,
                                                   double alpha, void* stream) {
  if (n_tiles < 0 || n_tiles > 0x7ffffff0) return tace_fail_msg("tace_seg_linear_presplit_frag_split: bad tile count");
  if (splits < 2 || splits > 64) return tace_fail_msg("tace_seg_linear_presplit_frag_split: 2..64 splits");
  if (n_tiles * splits > 0x7ffffff0 || n_tiles > 0x7ffffff)
    return tace_fail_msg("tace_seg_linear_presplit_frag_split: too many work items");
  if (n_tiles == 0) return 0;
  if (!x || !y || !w_frag || !tiles || !contribs || !partials)
    return tace_fail_msg("tace_seg_linear_presplit_frag_split: null pointer");
  if (addend && alpha == 0.0) return tace_fail_msg("tace_seg_linear_presplit_frag_split: an addend needs alpha != 0");
  if ((((uintptr_t)w_frag) & 15) != 0 || (((uintptr_t)partials) & 15) != 0)
    return tace_fail_msg("tace_seg_linear_presplit_frag_split: weights and partials must be 16-byte aligned");
  if (partial_elems < n_tiles * splits * 16384)
    return tace_fail_msg("tace_seg_linear_presplit_frag_split: partials hold fewer than n_tiles * splits * 16384 floats");
  const int64_t items = n_tiles * splits;
  const int per = (int)((items + 7) / 8);
  const dim3 g((unsigned)(8 * per)), b(256);
  if (aligned && (((uintptr_t)x) & 15) == 0)
    hipLaunchKernelGGL((k_seg_linear_bx3f<true, true>), g, b, 0, (hipStream_t)stream, x, y, addend,
                       (const unsigned short*)w_frag, bias, tiles, contribs, (float)alpha, (int)n_tiles, per,
                       (int)splits, partials);
  else
    hipLaunchKernelGGL((k_seg_linear_bx3f<false, true>), g, b, 0, (hipStream_t)stream, x, y, addend,
                       (const unsigned short*)w_frag, bias, tiles, contribs, (float)alpha, (int)n_tiles, per,
                       (int)splits, partials);
  if (int rc = tace_check_launch("tace_seg_linear_presplit_frag_split")) return rc;
  hipLaunchKernelGGL(k_seg_split_sum, dim3((unsigned)(16 * n_tiles)), dim3(256), 0, (hipStream_t)stream, y, addend, bias,
                     tiles, (const float*)partials, (int)splits, (float)alpha);
  return tace_check_launch("tace_seg_linear_presplit_frag_split");
}

extern "C" int32_t tace_seg_linear_ks_rows(int32_t k) { return k < 0 ? 0 : k <= 128 ? 128 : k <= 256 ? 64 : 0; }

extern "C" int tace_seg_linear_presplit_ks(const float* x, float* y, const float* addend, const uint16_t* w_frag,
                                           const float* bias,
                                           const int64_t* tasks, int64_t n_tasks, int32_t task_rows, double alpha,
                                           void* stream) {
  if (task_rows != 128 && task_rows != 64)
    return tace_fail_msg("tace_seg_linear_presplit_ks: tasks of 128 rows (k <= 128) or 64 rows (k <= 256)");
  if (n_tasks < 0 || n_tasks > 0x7ffffff0) return tace_fail_msg("tace_seg_linear_presplit_ks: bad task count");
  if (n_tasks == 0) return 0;
  if (!x || !y || !w_frag || !tasks) return tace_fail_msg("tace_seg_linear_presplit_ks: null pointer");
  if (addend && alpha == 0.0) return tace_fail_msg("tace_seg_linear_presplit_ks: an addend needs alpha != 0");
  if ((((uintptr_t)w_frag) & 15) != 0)
    return tace_fail_msg("tace_seg_linear_presplit_ks: the fragment-order weights must be 16-byte aligned");
  const int per = (int)((n_tasks + 7) / 8);
  if (task_rows == 128)
    hipLaunchKernelGGL((k_seg_linear_ks<128, 128>), dim3((unsigned)(8 * per)), dim3(KS_THREADS), 0, (hipStream_t)stream,
                       x, y, addend, (const unsigned short*)w_frag, bias, tasks, (float)alpha, (int)n_tasks, per);
  else
    hipLaunchKernelGGL((k_seg_linear_ks<64, 256>), dim3((unsigned)(8 * per)), dim3(KS_THREADS), 0, (hipStream_t)stream,
                       x, y, addend, (const unsigned short*)w_frag, bias, tasks, (float)alpha, (int)n_tasks, per);
  return tace_check_launch("tace_seg_linear_presplit_ks");
}

extern "C" int tace_seg_linear(int dtype, int32_t tile_rows, int32_t tile_cols, const void* x, void* y,
                               const void* addend, const void* w, const void* bias, const int64_t* tiles, int64_t n_tiles,
                               const int64_t* contribs, const double* scales, double alpha, void* stream) {
  if (n_tiles < 0 || n_tiles > 0x7ffffff0) return tace_fail_msg("tace_seg_linear: bad tile count");
  const int tr = tile_rows, tc = tile_cols;
  const bool mfma = dtype == TACE_F32 && tr == 128 && tc == 128;
  if (!(mfma || ((dtype == TACE_F32 || dtype == TACE_F64) && tr == 64 && tc == 64)))
    return tace_fail_msg("tace_seg_linear: tiles must be 128x128 (float32) or 64x64");
  if (n_tiles == 0) return 0;
  if (!x || !y || !w || !tiles || !contribs || !scales) return tace_fail_msg("tace_seg_linear: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)n_tiles), block(256);
  if (mfma) {
    const int per = (int)((n_tiles + 7) / 8);
    const dim3 g8((unsigned)(8 * per));
    hipLaunchKernelGGL(k_seg_linear_bf16x3, g8, block, 0, s, (const float*)x, (float*)y, (const float*)addend,
                       (const float*)w,
                       (const float*)bias, tiles, contribs, scales, (float)alpha, (int)n_tiles, per);
  } else if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_seg_linear<float>, grid, block, 0, s, (const float*)x, (float*)y, (const float*)addend,
                       (const float*)w,
                       (const float*)bias, tiles, contribs, scales, (float)alpha);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_seg_linear<double>, grid, block, 0, s, (const double*)x, (double*)y,
                       (const double*)addend, (const double*)w,
                       (const double*)bias, tiles, contribs, scales, alpha);
  else
    return tace_fail_msg("tace_seg_linear: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_seg_linear");
}
