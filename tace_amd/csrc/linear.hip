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
// Output: y[tile] = alpha * (sum_c scale_c x_c[tile rows] @ B_c + bias), every
// element of every tile written (no accumulation into y).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tace_hip.h"

int tace_fail_msg(const char* msg);   // tace_hip.hip
int tace_check_launch(const char* what);

namespace {

constexpr int TM = 64, TN = 64, TK = 16, PAD = 4;

// 256 threads = 16 x 16; thread (ty, tx) owns rows ty*4..ty*4+3 and columns
// tx*4..tx*4+3 of the tile.  A and B stage through LDS k-major (As[k][row],
// Bs[k][col]) so the inner product reads one 4-vector of each per k.
template <typename T>
__global__ __launch_bounds__(256) void k_seg_linear(const T* __restrict__ x, T* __restrict__ y,
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
      if (col < n) y[out_base + (int64_t)r * n + col] = alpha * (acc[i][j] + bv[j]);
    }
  }
}

// float32 on MFMA: 4 waves in a 2 x 2 grid, each owning WM x WN blocks of
// 16 x 16 (v_mfma_f32_16x16x4f32), so a tile is (32 WM) x (32 WN); the
// library runs 128 x 128 (4, 4) at 2 waves per SIMD.  (256 x 128 and 128 x 256
// tiles halve the weight or input re-reads of config 4's linears but need
// ~350 registers per lane, 1 wave per SIMD, and measured 12-20% slower.)  A stages through LDS k-contiguous (As[row][k]) in chunks of 32
// k; since the sum over k is order free, in MFMA step s lane l supplies
// A[row][4 (l/16) + s] of a 16-k half, so it reads its four k values of a
// fragment as one 16-byte LDS load.  B keeps the layout of its source:
// k-contiguous (Bt[col][k], one 16-byte read per fragment) for the input
// gradient, whose W^T rows are W's k-contiguous rows, and column-contiguous
// (Bn[k][col], four 4-byte reads) for the forward, whose W [k, n] rows run
// along the columns -- every global load is a 16-byte load and no staging
// store transposes.  The next chunk's global loads are issued before the
// current chunk's MFMAs and land in registers, so memory latency overlaps the
// matrix work.  Tiles are taken XCD-grouped: workgroup b runs tile (b % 8) *
// per + b / 8, so XCD k works through a contiguous stretch of the table (the
// column tiles of one row tile, the row tiles of one species' weight) and
// shares them in its L2.
constexpr int MK = 32, MPAD = 4, NPAD = 4;
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

template <int R>
__device__ __forceinline__ void seg_store_k(float* lds, int stride, int t, const f4* v, float sc) {
#pragma unroll
  for (int rr = 0; rr < R / 128; ++rr)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *(f4*)&lds[((t >> 1) + 128 * rr) * stride + 16 * (t & 1) + 4 * q] = v[4 * rr + q] * sc;
}

// 32 k rows x Cn columns of W [k, n] (columns c0 ..): thread t holds k row
// t % 32 and columns 4 (t/32) + 32 q + 128 cc (q < 4, cc < Cn/128)
template <int Cn>
__device__ __forceinline__ void seg_load_n(const float* __restrict__ wb, int k, int n, int c0, int k0, bool vec, int t,
                                           f4* v) {
  const int kk = k0 + (t & 31), cb = c0 + 4 * (t >> 5);
  const float* p = wb + (int64_t)kk * n + cb;
#pragma unroll
  for (int cc = 0; cc < Cn / 128; ++cc)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int left = n - (cb + 32 * q + 128 * cc);
      v[4 * cc + q] = seg_ld4(p + 32 * q + 128 * cc, kk < k && vec && left >= 4, kk < k && left > 0, left);
    }
}

template <int Cn>
__device__ __forceinline__ void seg_store_n(float* lds, int t, const f4* v, float sc) {
#pragma unroll
  for (int cc = 0; cc < Cn / 128; ++cc)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *(f4*)&lds[(t & 31) * (Cn + NPAD) + 4 * (t >> 5) + 32 * q + 128 * cc] = v[4 * cc + q] * sc;
}

template <int WM, int WN>
__global__ __launch_bounds__(256) void k_seg_linear_mfma(const float* __restrict__ x, float* __restrict__ y,
                                                         const float* __restrict__ w, const float* __restrict__ bias,
                                                         const int64_t* __restrict__ tiles,
                                                         const int64_t* __restrict__ contribs,
                                                         const double* __restrict__ scales, float alpha,
                                                         int n_tiles, int per) {
  constexpr int TR = 32 * WM, TC = 32 * WN, BT = MK + MPAD;
  constexpr int BS = (TC * BT > MK * (TC + NPAD)) ? TC * BT : MK * (TC + NPAD);
  __shared__ float As[TR * BT];
  __shared__ float Bs[BS];   // Bt[TC][MK + MPAD] or Bn[MK][TC + NPAD]
  const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (tile >= n_tiles) return;
  const int64_t* td = tiles + 8 * (int64_t)tile;
  const int64_t out_base = td[0];
  const int rows = (int)td[1], n = (int)td[2], c0 = (int)td[3];
  const int64_t bias_off = td[4];
  const int cb = (int)td[5], ce = (int)td[6];
  const int t = (int)threadIdx.x, lane = t & 63, wv = t >> 6;
  const int wr = (wv >> 1) * 16 * WM, wc = (wv & 1) * 16 * WN;   // the wave's block of the tile
  const int fr = lane & 15, fg = lane >> 4;                        // fragment row/col, k group
  constexpr int NA = TR / 32, NB = TC / 32;   // f4 per thread per chunk
  f4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  for (int c = cb; c < ce; ++c) {
    const int64_t* cd = contribs + 4 * (int64_t)c;
    const float* __restrict__ xa = x + cd[0];
    const int k = (int)cd[1];
    const float* __restrict__ wb = w + cd[2];
    const bool trans = cd[3] != 0;
    const float sc = (float)scales[c];
    const bool xvec = ((((uintptr_t)xa) & 15) == 0) && ((k & 3) == 0);
    const bool wvec = ((((uintptr_t)wb) & 15) == 0) && (((trans ? k : n) & 3) == 0) && ((c0 & 3) == 0);
    const float* __restrict__ wt = wb + (int64_t)c0 * k;   // W^T tile rows (trans)
    f4 a[NA], b[NB];
    seg_load_k<TR>(xa, k, 0, rows, xvec, t, a);
    if (trans) seg_load_k<TC>(wt, k, 0, n - c0, wvec, t, b);
    else seg_load_n<TC>(wb, k, n, c0, 0, wvec, t, b);
    for (int k0 = 0; k0 < k; k0 += MK) {
      seg_store_k<TR>(As, BT, t, a, 1.f);
      if (trans) seg_store_k<TC>(Bs, BT, t, b, sc);
      else seg_store_n<TC>(Bs, t, b, sc);
      __syncthreads();
      if (k0 + MK < k) {   // next chunk in flight during this chunk's MFMAs
        seg_load_k<TR>(xa, k, k0 + MK, rows, xvec, t, a);
        if (trans) seg_load_k<TC>(wt, k, k0 + MK, n - c0, wvec, t, b);
        else seg_load_n<TC>(wb, k, n, c0, k0 + MK, wvec, t, b);
      }
#pragma unroll
      for (int h = 0; h < MK; h += 16) {
        f4 af[WM], bf[WN];
#pragma unroll
        for (int i = 0; i < WM; ++i) af[i] = *(const f4*)&As[(wr + 16 * i + fr) * BT + h + 4 * fg];
        if (trans) {
#pragma unroll
          for (int j = 0; j < WN; ++j) bf[j] = *(const f4*)&Bs[(wc + 16 * j + fr) * BT + h + 4 * fg];
        } else {
#pragma unroll
          for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) bf[j][s2] = Bs[(h + 4 * fg + s2) * (TC + NPAD) + wc + 16 * j + fr];
        }
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
          for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s2], bf[j][s2], acc[i][j], 0, 0, 0);
      }
      __syncthreads();
    }
  }
  // D lane l, register q of block (i, j) = tile row wr + 16 i + 4 (l/16) + q, column wc + 16 j + l%16
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
        if (r < rows) y[out_base + (int64_t)r * n + col] = alpha * (acc[i][j][q] + bv);
      }
  }
}

}  // namespace

extern "C" int tace_seg_linear(int dtype, int32_t tile_rows, int32_t tile_cols, const void* x, void* y,
                               const void* w, const void* bias, const int64_t* tiles, int64_t n_tiles,
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
    hipLaunchKernelGGL((k_seg_linear_mfma<4, 4>), g8, block, 0, s, (const float*)x, (float*)y, (const float*)w,
                       (const float*)bias, tiles, contribs, scales, (float)alpha, (int)n_tiles, per);
  } else if (dtype == TACE_F32)
    hipLaunchKernelGGL(k_seg_linear<float>, grid, block, 0, s, (const float*)x, (float*)y, (const float*)w,
                       (const float*)bias, tiles, contribs, scales, (float)alpha);
  else if (dtype == TACE_F64)
    hipLaunchKernelGGL(k_seg_linear<double>, grid, block, 0, s, (const double*)x, (double*)y, (const double*)w,
                       (const double*)bias, tiles, contribs, scales, alpha);
  else
    return tace_fail_msg("tace_seg_linear: dtype must be TACE_F32 or TACE_F64");
  return tace_check_launch("tace_seg_linear");
}
