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
// (row-major, scale folded in); the last hidden activations h [E, 64]
// row-major (the A operand of the last layer's GEMM).  Nothing is saved for
// the backward: it recomputes the pre-activations from the radial basis.
//
// float32 runs the layers on MFMA (k_mlp_fwd_mfma / k_mlp_bwd_mfma): per
// 32-edge block a wavefront multiplies [32 x K] activations by the [K x 64]
// weights with v_mfma_f32_32x32x2f32 (weights staged once per workgroup in
// LDS), applies SiLU (or its derivative) to the accumulators and passes the
// result to the next layer through a per-wavefront LDS tile (the accumulator
// layout holds a column per lane, the A operand needs a row); h is stored
// straight from the accumulators, two 128-byte row segments per store.  The per-thread kernels below stay for float64.
#include <hip/hip_runtime.h>

#include "bf16x3.h"
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

// pre-activation z of layer `upto` of edge e (the forward recomputed from the
// radial basis; a_ holds the activations of the layer before)
template <typename T>
__device__ __forceinline__ void mlp_forward_to(const T* __restrict__ r, int n_in, int upto, const T* __restrict__ w,
                                               T* __restrict__ z, T* __restrict__ a_) {
#pragma unroll
  for (int j = 0; j < W; ++j) z[j] = T(0);
  for (int k = 0; k < n_in; ++k) {
    const T a = r[k];
#pragma unroll
    for (int j = 0; j < W; ++j) z[j] += a * w[k * W + j];
  }
  int off = n_in * W;
  for (int l = 0; l < upto; ++l) {
#pragma unroll
    for (int j = 0; j < W; ++j) {
      a_[j] = z[j] * sigm(z[j]);
      z[j] = T(0);
    }
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const T a = a_[k];
#pragma unroll
      for (int j = 0; j < W; ++j) z[j] += a * w[off + k * W + j];
    }
    off += W * W;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_mlp_fwd(const T* __restrict__ radial, int64_t E, int n_in, int n_layers,
                                                 const T* __restrict__ wg, T* __restrict__ h) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  T a_[W], z[W];
  mlp_forward_to<T>(radial + e * n_in, n_in, n_layers - 1, wg, z, a_);
#pragma unroll
  for (int j = 0; j < W; ++j) h[e * W + j] = z[j] * sigm(z[j]);
}

// backward to the radial basis: g_z = g_h silu'(z), g_h(prev) = W g_z, with
// each layer's pre-activation recomputed from the radial basis (nothing is
// saved between the forward and the backward)
template <typename T>
__global__ __launch_bounds__(256) void k_mlp_bwd(const T* __restrict__ radial, const T* __restrict__ gh, int64_t E,
                                                 int n_in, int n_layers, const T* __restrict__ wg,
                                                 T* __restrict__ g_radial) {
  const T* __restrict__ w = wg;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  T g[W], z[W], a_[W];
#pragma unroll
  for (int j = 0; j < W; ++j) g[j] = gh[e * W + j];
  for (int l = n_layers - 1; l >= 0; --l) {
    mlp_forward_to<T>(radial + e * n_in, n_in, l, wg, z, a_);
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const T s = sigm(z[j]);
      g[j] *= s * (T(1) + z[j] * (T(1) - s));
    }
    if (l == 0) break;
    const int off = n_in * W + (l - 1) * W * W;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      T acc = T(0);
#pragma unroll
      for (int j = 0; j < W; ++j) acc += w[off + k * W + j] * g[j];
      a_[k] = acc;
    }
#pragma unroll
    for (int k = 0; k < W; ++k) g[k] = a_[k];
  }
  for (int k = 0; k < n_in; ++k) {
    T acc = T(0);
#pragma unroll
    for (int j = 0; j < W; ++j) acc += w[k * W + j] * g[j];
    g_radial[e * n_in + k] = acc;
  }
}

// ------------------------------------------------- hidden layers on MFMA --
typedef float f16_t __attribute__((ext_vector_type(16)));
constexpr int TSTRIDE = 68;  // LDS tile row stride (16-byte aligned rows)

// accumulator r of lane (i, q) in the 32 x 32 output layout: row
// 8 (r / 4) + 4 q + r % 4, column i
__device__ __forceinline__ int acc_row(int r, int q) { return 8 * (r >> 2) + 4 * q + (r & 3); }

// the [32 x 64] accumulator pair -> LDS tile -> A fragment (lane (i, q) of
// k-step s holds row i, k = 32 q + s)
__device__ __forceinline__ void tile_to_afrag(const f16_t* acc, float* __restrict__ T, int i, int q, float* a) {
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) T[acc_row(r, q) * TSTRIDE + 32 * cb + i] = acc[cb][r];
  __builtin_amdgcn_wave_barrier();
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v* tp = reinterpret_cast<const f4v*>(T + i * TSTRIDE + 32 * q);
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const f4v t = tp[v];
    a[4 * v] = t[0]; a[4 * v + 1] = t[1]; a[4 * v + 2] = t[2]; a[4 * v + 3] = t[3];
  }
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ float silu_f(float z) { return z * (1.0f / (1.0f + expf(-z))); }
__device__ __forceinline__ float dsilu_f(float z) {
  const float s = 1.0f / (1.0f + expf(-z));
  return s * (1.0f + z * (1.0f - s));
}

// LDS: the weights with row stride WSTR (layer 0: K0p = n_in rounded up to
// even rows, zero past n_in; hidden layers: 64 rows each), then one tile
// [32 x TSTRIDE] per wavefront.  With the odd stride one copy serves both
// orientations without bank conflicts: the forward reads W[k][32 cb + lane],
// the backward W[32 cb + lane][j].
constexpr int WSTR = 65;

__host__ __device__ __forceinline__ int mlp_lds_weights(int n_in, int n_layers) {
  return (((n_in + 1) & ~1) + (n_layers - 1) * 64) * WSTR;
}

__device__ __forceinline__ void mlp_stage_weights(const float* __restrict__ wg, int n_in, int n_layers,
                                                  float* __restrict__ smem) {
  const int K0p = (n_in + 1) & ~1, rows = K0p + (n_layers - 1) * 64;
  for (int t = (int)threadIdx.x; t < rows * 64; t += 256) {
    const int r = t >> 6, j = t & 63;
    smem[r * WSTR + j] = r < K0p ? (r < n_in ? wg[r * 64 + j] : 0.0f) : wg[(n_in + r - K0p) * 64 + j];
  }
}

// pre-activation z of layer `upto` of the 32-edge block at e0, in the
// accumulator layout (first layer: A = radial rows, lane half q holds
// k = S0 q + s; then A = the previous activations through the LDS tile)
__device__ __forceinline__ void mlp_block_z(const float* __restrict__ radial, int64_t E, int n_in, int64_t e0,
                                            int upto, const float* __restrict__ smem, float* __restrict__ T, int i,
                                            int q, f16_t* z) {
  const int K0p = (n_in + 1) & ~1, S0 = K0p >> 1;
  const int64_t er = e0 + i;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) z[cb][r] = 0.0f;
  for (int s = 0; s < S0; ++s) {
    const int k = S0 * q + s;
    const float av = er < E && k < n_in ? radial[er * n_in + k] : 0.0f;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
      z[cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, smem[k * WSTR + 32 * cb + i], z[cb], 0, 0, 0);
  }
  for (int l = 1; l <= upto; ++l) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) z[cb][r] = silu_f(z[cb][r]);
    float a[32];
    tile_to_afrag(z, T, i, q, a);
    const float* __restrict__ Wl = smem + (K0p + (l - 1) * 64) * WSTR;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) z[cb][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; ++s)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        z[cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], Wl[(32 * q + s) * WSTR + 32 * cb + i], z[cb], 0, 0, 0);
  }
}

// pre-activations z[0 .. NL-1] of the 32-edge block at e0 (all layers kept
// for the backward)
template <int NL>
__device__ __forceinline__ void mlp_block_forward(const float* __restrict__ radial, int64_t E, int n_in, int64_t e0,
                                                  const float* __restrict__ smem, float* __restrict__ T, int i, int q,
                                                  f16_t (*z)[2]) {
  mlp_block_z(radial, E, n_in, e0, 0, smem, T, i, q, z[0]);
  const int K0p = (n_in + 1) & ~1;
#pragma unroll
  for (int l = 1; l < NL; ++l) {
    f16_t act[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) act[cb][r] = silu_f(z[l - 1][cb][r]);
    float a[32];
    tile_to_afrag(act, T, i, q, a);
    const float* __restrict__ Wl = smem + (K0p + (l - 1) * 64) * WSTR;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) z[l][cb][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; ++s)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        z[l][cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], Wl[(32 * q + s) * WSTR + 32 * cb + i], z[l][cb], 0, 0, 0);
  }
}

template <int NL>
__global__ __launch_bounds__(256) void k_mlp_fwd_mfma(const float* __restrict__ radial, int64_t E, int n_in,
                                                      const float* __restrict__ wg, float* __restrict__ h) {
  extern __shared__ float smem[];
  mlp_stage_weights(wg, n_in, NL, smem);
  __syncthreads();
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6, i = lane & 31, q = lane >> 5;
  float* __restrict__ T = smem + mlp_lds_weights(n_in, NL) + wave * 32 * TSTRIDE;
  const int64_t nblk = (E + 31) / 32;
  for (int64_t blk = (int64_t)blockIdx.x * 4 + wave; blk < nblk; blk += (int64_t)gridDim.x * 4) {
    const int64_t e0 = blk * 32;
    f16_t z[2];
    mlp_block_z(radial, E, n_in, e0, NL - 1, smem, T, i, q, z);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t e = e0 + acc_row(r, q);
        if (e < E) h[e * 64 + 32 * cb + i] = silu_f(z[cb][r]);
      }
  }
}

// the backward recomputes the block's pre-activations (one forward pass on
// MFMA, all layers kept in registers) instead of saving 64 floats per edge
// and layer in the forward.  Measured against the saved-z version: 0.77 vs
// 0.68 ms backward, 0.37 vs 0.42 ms forward; recomputing each layer where it
// is needed (one layer in registers, 2 wavefronts per SIMD) measured 0.90 ms.
template <int NL>
__global__ __launch_bounds__(256) void k_mlp_bwd_mfma(const float* __restrict__ radial, const float* __restrict__ gh,
                                                      int64_t E, int n_in, const float* __restrict__ wg,
                                                      float* __restrict__ g_radial) {
  extern __shared__ float smem[];
  mlp_stage_weights(wg, n_in, NL, smem);
  __syncthreads();
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6, i = lane & 31, q = lane >> 5;
  const int K0p = (n_in + 1) & ~1;
  float* __restrict__ T = smem + mlp_lds_weights(n_in, NL) + wave * 32 * TSTRIDE;
  const int64_t nblk = (E + 31) / 32;
  for (int64_t blk = (int64_t)blockIdx.x * 4 + wave; blk < nblk; blk += (int64_t)gridDim.x * 4) {
    const int64_t e0 = blk * 32;
    f16_t z[NL][2];
    mlp_block_forward<NL>(radial, E, n_in, e0, smem, T, i, q, z);
    f16_t g[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t e = e0 + acc_row(r, q);
        g[cb][r] = e < E ? gh[e * 64 + 32 * cb + i] : 0.0f;
      }
#pragma unroll
    for (int l = NL - 1; l >= 0; --l) {
      // g_z = g_a silu'(z_l), then A = g_z through the tile
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) g[cb][r] *= dsilu_f(z[l][cb][r]);
      float a[32];
      tile_to_afrag(g, T, i, q, a);
      if (l == 0) {
        // g_radial[e][k] = sum_j g_z[e][j] W_0[k][j]: B[j][k = lane] = W_0[lane][j]
        f16_t acc = {};
#pragma unroll
        for (int s = 0; s < 32; ++s)
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], i < n_in ? smem[i * WSTR + 32 * q + s] : 0.0f, acc, 0, 0,
                                                     0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t e = e0 + acc_row(r, q);
          if (e < E && i < n_in) g_radial[e * n_in + i] = acc[r];
        }
      } else {
        // g_a[e][k] = sum_j g_z[e][j] W_l[k][j]: B[j][k] = W_l[k][j]
        const float* __restrict__ Wl = smem + (K0p + (l - 1) * 64) * WSTR;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
          for (int r = 0; r < 16; ++r) g[cb][r] = 0.0f;
#pragma unroll
        for (int s = 0; s < 32; ++s)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            g[cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], Wl[(32 * cb + i) * WSTR + 32 * q + s], g[cb], 0, 0, 0);
      }
    }
  }
}

// ------------------------------------------------------------- last layer --
// out[e, n] = alpha sum_k h[e, k] W[k, n] with K = 64 (the wide, linear last
// layer: E ~ 1e6 edges x N ~ 3e3 weights, output-write bound).  float32 runs
// on the bf16 MFMA (v_mfma_f32_32x32x16_bf16) with both operands split into
// three bf16 terms (bf16x3.h: exact split, six products, float32 rounding).
// Each wavefront owns 64 output columns (two 32-column blocks) and keeps the
// three terms of their 64 x 64 slice of W in registers as B fragments for its
// whole life; it then streams 32-edge blocks: A from h (one 128-byte row
// segment per lane, split once), 4 k-steps x 2 column blocks x 6 terms of
// MFMA, and the two 32 x 32 result tiles stored straight from the
// accumulators -- in the 32 x 32 output layout every store instruction writes
// two whole 128-byte row segments, so no transpose through LDS is needed; the
// stores are non-temporal (the output is streamed once to HBM).  K is
// permuted (lane half q of step s holds k = 32 q + 8 s .. + 7) so that a
// lane's A values are one contiguous row segment; B uses the same k for the
// same lane and item.  Workgroups (4 waves = 256 columns) that share an edge
// chunk are placed on one XCD (blockIdx round-robins over the 8 XCDs), so the
// chunk's h rows are read from HBM about once.
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void load_a_frag32(const float* __restrict__ h, int64_t er, int64_t E, int q, float* a) {
  if (er < E) {
    const f4_t* hp = reinterpret_cast<const f4_t*>(h + er * 64 + 32 * q);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const f4_t t = hp[v];
      a[4 * v] = t[0]; a[4 * v + 1] = t[1]; a[4 * v + 2] = t[2]; a[4 * v + 3] = t[3];
    }
  } else {
#pragma unroll
    for (int s = 0; s < 32; ++s) a[s] = 0.0f;
  }
}

__global__ __launch_bounds__(256) void k_mlp_out_f32(const float* __restrict__ h, const float* __restrict__ Wm,
                                                     int64_t E, int N, float alpha, int n_col_tiles,
                                                     int64_t n_chunks, int edges_per_chunk, float* __restrict__ out) {
  const int b = (int)blockIdx.x;
  const int64_t chunk = (int64_t)(b & 7) + 8 * (int64_t)((b >> 3) / n_col_tiles);
  const int ct = (b >> 3) % n_col_tiles;
  if (chunk >= n_chunks) return;
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int i = lane & 31, q = lane >> 5;
  const int col0 = ct * 256 + wave * 64;
  // B fragments: lane (i, q) of step s, item j holds W[32 q + 8 s + j][col0 + 32 cb + i]
  bx3_bf8 bw[4][2][3];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int c = col0 + 32 * cb + i;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = c < N ? Wm[(int64_t)(32 * q + 8 * s + j) * N + c] : 0.0f;
      bx3_split8(v, bw[s][cb]);
    }
  const int64_t e_begin = chunk * edges_per_chunk;
  const int64_t e_end = e_begin + edges_per_chunk < E ? e_begin + edges_per_chunk : E;
  float a[32];
  load_a_frag32(h, e_begin + i, E, q, a);
  for (int64_t e0 = e_begin; e0 < e_end; e0 += 32) {
    bx3_bf8 at[4][3];
#pragma unroll
    for (int s = 0; s < 4; ++s) bx3_split8(a + 8 * s, at[s]);
    // next block's A fragment in flight during this block's MFMAs
    load_a_frag32(h, e0 + 32 < e_end ? e0 + 32 + i : E, E, q, a);
    f16_t acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[cb][r] = 0.0f;
#pragma unroll
    for (int u = 0; u < 6; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at[s][BX3_TA[u]], bw[s][cb][BX3_TB[u]], acc[cb], 0, 0, 0);
    // accumulator r of lane (i, q): row 8 (r / 4) + 4 q + r % 4, column i
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int c = col0 + 32 * cb + i;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = e0 + 8 * (r >> 2) + 4 * q + (r & 3);
        if (row < e_end && c < N) __builtin_nontemporal_store(alpha * acc[cb][r], out + row * N + c);
      }
    }
  }
}

// The last layer's input gradient: g_h[e, c] = alpha sum_n g[e, n] W[c, n]
// (c < 64; g [E, N] is the gradient of the layer's output).  float32 on the
// bf16 MFMA (v_mfma_f32_32x32x16_bf16) with the exact three-term split of
// bf16x3.h.  One wavefront per 32 edges and all 64 columns (two 32-column
// blocks), four per workgroup; they stream N in 32-wide slabs: lane (i, q)
// reads g[e0 + i][k0 + 16 q .. + 15] (each row's 128-byte slab segment over
// the two lane halves), and the workgroup splits the slab of W (64 x 32, from
// L2) once into three bf16 planes in LDS, from which lane (i, q) reads
// W[32 cb + i][same k] -- step s item j of both operands is k = k0 + 16 q +
// 8 s + j.  The next slab's loads are issued before the current slab's
// MFMAs.  Read-bound on g.
__device__ __forceinline__ void mlp_ld16(const float* __restrict__ row, int k, int N, bool ok, bool vec, float* v) {
  if (ok && vec && k + 16 <= N) {
    const f4_t* p = reinterpret_cast<const f4_t*>(row + k);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f4_t t = p[u];
      v[4 * u] = t[0]; v[4 * u + 1] = t[1]; v[4 * u + 2] = t[2]; v[4 * u + 3] = t[3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = (ok && k + j < N) ? row[k + j] : 0.0f;
  }
}

__device__ __forceinline__ void mlp_ld8(const float* __restrict__ row, int k, int N, bool vec, float* v) {
  if (vec && k + 8 <= N) {
    const f4_t* p = reinterpret_cast<const f4_t*>(row + k);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const f4_t t = p[u];
      v[4 * u] = t[0]; v[4 * u + 1] = t[1]; v[4 * u + 2] = t[2]; v[4 * u + 3] = t[3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = k + j < N ? row[k + j] : 0.0f;
  }
}

// PAIRS: output row e is the gradient of a weight row shared by two edges
// (the two directions of a pair have the same length, hence the same radial
// weights): g row = g[ra[e]] + g[rb[e]] (rb[e] < 0: g[ra[e]] alone), summed
// in float32 before the split.
template <bool PAIRS>
__global__ __launch_bounds__(256) void k_mlp_out_bwd_f32(const float* __restrict__ g, const float* __restrict__ Wm,
                                                         int64_t E, int N, float alpha, float* __restrict__ gh,
                                                         const int* __restrict__ ra, const int* __restrict__ rb) {
  constexpr int BSTR = 40;                       // bf16 per LDS row: 32 k + 8 pad (80 bytes)
  __shared__ __attribute__((aligned(16))) unsigned short Bp[3 * 64 * BSTR];   // term p, column c, k
  const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6;
  const int i = lane & 31, q = lane >> 5;
  const int64_t e0 = ((int64_t)blockIdx.x * 4 + wave) * 32;
  const int64_t er = e0 + i;
  const bool rok = er < E;
  const bool vec = (N & 3) == 0;
  const float* __restrict__ grow = g + (PAIRS ? (rok ? (int64_t)ra[er] : 0) : (rok ? er : 0)) * (int64_t)N;
  const int rbe = PAIRS && rok ? rb[er] : -1;
  const float* __restrict__ grow2 = g + (rbe >= 0 ? (int64_t)rbe : 0) * (int64_t)N;
  // the slab's W[c][k0 + kk .. + 7] for c = t / 4, kk = 8 (t % 4), split once per workgroup
  const int wc = t >> 2, wk = 8 * (t & 3);
  const float* __restrict__ wrow = Wm + (int64_t)wc * N;
  f16_t acc[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[cb][r] = 0.0f;
  float a[16], w[8], a2[16];
  mlp_ld16(grow, 16 * q, N, rok, vec, a);
  if (PAIRS) mlp_ld16(grow2, 16 * q, N, rbe >= 0, vec, a2);
  mlp_ld8(wrow, wk, N, vec, w);
  for (int k0 = 0; k0 < N; k0 += 32) {
    bx3_bf8 wt[3];
    bx3_split8(w, wt);
#pragma unroll
    for (int p = 0; p < 3; ++p) *(bx3_bf8*)&Bp[(p * 64 + wc) * BSTR + wk] = wt[p];
    if (PAIRS) {
#pragma unroll
      for (int j = 0; j < 16; ++j) a[j] += a2[j];
    }
    bx3_bf8 at[2][3];
#pragma unroll
    for (int s = 0; s < 2; ++s) bx3_split8(a + 8 * s, at[s]);
    __syncthreads();
    if (k0 + 32 < N) {   // next slab in flight during this slab's MFMAs
      mlp_ld16(grow, k0 + 32 + 16 * q, N, rok, vec, a);
      if (PAIRS) mlp_ld16(grow2, k0 + 32 + 16 * q, N, rbe >= 0, vec, a2);
      mlp_ld8(wrow, k0 + 32 + wk, N, vec, w);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        bx3_bf8 bt[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) bt[p] = *(const bx3_bf8*)&Bp[(p * 64 + 32 * cb + i) * BSTR + 16 * q + 8 * s];
#pragma unroll
        for (int u = 0; u < 6; ++u)
          acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at[s][BX3_TA[u]], bt[BX3_TB[u]], acc[cb], 0, 0, 0);
      }
    __syncthreads();
  }
  // accumulator r of lane (i, q): row 8 (r / 4) + 4 q + r % 4, column 32 cb + i
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = e0 + 8 * (r >> 2) + 4 * q + (r & 3);
      if (row < E) gh[row * 64 + 32 * cb + i] = alpha * acc[cb][r];
    }
}

size_t mlp_lds_bytes(int n_in, int n_layers) {
  return sizeof(float) * ((size_t)mlp_lds_weights(n_in, n_layers) + 4 * 32 * TSTRIDE);
}

// 4 wavefronts per workgroup, one 32-edge block per wavefront and pass
dim3 mlp_mfma_grid(int64_t E) {
  const int64_t wgs = ((E + 31) / 32 + 3) / 4;
  return dim3((unsigned)(wgs < 2048 ? (wgs > 0 ? wgs : 1) : 2048));
}

// dynamic LDS above the 64 KB default (the limit is per kernel and process)
int mlp_lds_attr(const void* fn, size_t bytes) {
  if (bytes <= 65536) return 0;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess)
    return tace_fail_msg("radial MLP: cannot raise the kernel's dynamic LDS limit");
  return 0;
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
                        const void* weights, void* h, void* stream) {
  if (mlp_checks("tace_radial_mlp_fwd", n_edges, n_in, n_layers)) return -1;
  if (n_edges == 0) return 0;
  if (!radial || !weights || !h) return tace_fail_msg("tace_radial_mlp_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges + 255) / 256)), b(256);
  if (dtype == TACE_F32) {
    const size_t lds = mlp_lds_bytes(n_in, n_layers);
    const float *r = (const float*)radial, *w = (const float*)weights;
    float* o = (float*)h;
#define MLP_FWD(NL)                                                                                   \
  if (mlp_lds_attr((const void*)k_mlp_fwd_mfma<NL>, lds)) return -1;                                  \
  hipLaunchKernelGGL(k_mlp_fwd_mfma<NL>, mlp_mfma_grid(n_edges), b, lds, s, r, n_edges, n_in, w, o)
    switch (n_layers) {
      case 1: MLP_FWD(1); break;
      case 2: MLP_FWD(2); break;
      case 3: MLP_FWD(3); break;
      default: MLP_FWD(4); break;
    }
#undef MLP_FWD
  } else if (dtype == TACE_F64) {
    hipLaunchKernelGGL(k_mlp_fwd<double>, g, b, 0, s, (const double*)radial, n_edges, n_in, n_layers,
                       (const double*)weights, (double*)h);
  } else {
    return tace_fail_msg("tace_radial_mlp_fwd: dtype must be TACE_F32 or TACE_F64");
  }
  return tace_check_launch("tace_radial_mlp_fwd");
}

int tace_radial_mlp_bwd(int dtype, const void* radial, const void* g_h, int64_t n_edges, int32_t n_in,
                        int32_t n_layers, const void* weights, void* g_radial, void* stream) {
  if (mlp_checks("tace_radial_mlp_bwd", n_edges, n_in, n_layers)) return -1;
  if (n_edges == 0) return 0;
  if (!radial || !g_h || !weights || !g_radial) return tace_fail_msg("tace_radial_mlp_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)((n_edges + 255) / 256)), b(256);
  if (dtype == TACE_F32) {
    const size_t lds = mlp_lds_bytes(n_in, n_layers);
    const float *r = (const float*)radial, *gg = (const float*)g_h, *w = (const float*)weights;
    float* o = (float*)g_radial;
#define MLP_BWD(NL)                                                                                   \
  if (mlp_lds_attr((const void*)k_mlp_bwd_mfma<NL>, lds)) return -1;                                  \
  hipLaunchKernelGGL(k_mlp_bwd_mfma<NL>, mlp_mfma_grid(n_edges), b, lds, s, r, gg, n_edges, n_in, w, o)
    switch (n_layers) {
      case 1: MLP_BWD(1); break;
      case 2: MLP_BWD(2); break;
      case 3: MLP_BWD(3); break;
      default: MLP_BWD(4); break;
    }
#undef MLP_BWD
  } else if (dtype == TACE_F64) {
    hipLaunchKernelGGL(k_mlp_bwd<double>, g, b, 0, s, (const double*)radial, (const double*)g_h, n_edges, n_in,
                       n_layers, (const double*)weights, (double*)g_radial);
  } else {
    return tace_fail_msg("tace_radial_mlp_bwd: dtype must be TACE_F32 or TACE_F64");
  }
  return tace_check_launch("tace_radial_mlp_bwd");
}

int tace_radial_mlp_out_f32(const float* h, const float* weight, int64_t n_edges, int32_t n_out, float alpha,
                            float* out, void* stream) {
  if (n_edges < 0 || n_out <= 0) return tace_fail_msg("tace_radial_mlp_out_f32: bad sizes");
  if (n_edges == 0) return 0;
  if (!h || !weight || !out) return tace_fail_msg("tace_radial_mlp_out_f32: null pointer");
  if (((uintptr_t)h & 15) != 0) return tace_fail_msg("tace_radial_mlp_out_f32: h must be 16-byte aligned");
  // 1,024 edges per chunk, fewer (down to 128) when that leaves fewer than
  // 2,048 workgroups: small systems still fill the GPU
  const int n_col_tiles = (n_out + 255) / 256;
  int edges_per_chunk = 1024;
  while (edges_per_chunk > 128 && n_col_tiles * ((n_edges + edges_per_chunk - 1) / edges_per_chunk) < 2048)
    edges_per_chunk >>= 1;
  const int64_t n_chunks = (n_edges + edges_per_chunk - 1) / edges_per_chunk;
  const int64_t n_wg = n_col_tiles * ((n_chunks + 7) / 8) * 8;
  if (n_wg > INT32_MAX) return tace_fail_msg("tace_radial_mlp_out_f32: too many edges");
  hipLaunchKernelGGL(k_mlp_out_f32, dim3((unsigned)n_wg), dim3(256), 0, (hipStream_t)stream, h, weight, n_edges, n_out,
                     alpha, n_col_tiles, n_chunks, edges_per_chunk, out);
  return tace_check_launch("tace_radial_mlp_out_f32");
}

int tace_radial_mlp_out_bwd_f32(const float* g_out, const float* weight, int64_t n_edges, int32_t n_out, float alpha,
                                float* g_h, void* stream) {
  if (n_edges < 0 || n_out <= 0) return tace_fail_msg("tace_radial_mlp_out_bwd_f32: bad sizes");
  if (n_edges == 0) return 0;
  if (!g_out || !weight || !g_h) return tace_fail_msg("tace_radial_mlp_out_bwd_f32: null pointer");
  if ((n_out & 3) == 0 && ((((uintptr_t)g_out) | ((uintptr_t)weight)) & 15) != 0)
    return tace_fail_msg("tace_radial_mlp_out_bwd_f32: g_out and weight must be 16-byte aligned");
  const int64_t n_wg = (n_edges + 127) / 128;
  if (n_wg > INT32_MAX) return tace_fail_msg("tace_radial_mlp_out_bwd_f32: too many edges");
  hipLaunchKernelGGL(k_mlp_out_bwd_f32<false>, dim3((unsigned)n_wg), dim3(256), 0, (hipStream_t)stream, g_out,
                     weight, n_edges, n_out, alpha, g_h, nullptr, nullptr);
  return tace_check_launch("tace_radial_mlp_out_bwd_f32");
}

int tace_radial_mlp_out_bwd_pairs_f32(const float* g_out, const int32_t* rows_a, const int32_t* rows_b,
                                      int64_t n_rows, int32_t n_out, float alpha, const float* weight, float* g_h,
                                      void* stream) {
  if (n_rows < 0 || n_out <= 0) return tace_fail_msg("tace_radial_mlp_out_bwd_pairs_f32: bad sizes");
  if (n_rows == 0) return 0;
  if (!g_out || !rows_a || !rows_b || !weight || !g_h)
    return tace_fail_msg("tace_radial_mlp_out_bwd_pairs_f32: null pointer");
  if ((n_out & 3) == 0 && ((((uintptr_t)g_out) | ((uintptr_t)weight)) & 15) != 0)
    return tace_fail_msg("tace_radial_mlp_out_bwd_pairs_f32: g_out and weight must be 16-byte aligned");
  const int64_t n_wg = (n_rows + 127) / 128;
  if (n_wg > INT32_MAX) return tace_fail_msg("tace_radial_mlp_out_bwd_pairs_f32: too many rows");
  hipLaunchKernelGGL(k_mlp_out_bwd_f32<true>, dim3((unsigned)n_wg), dim3(256), 0, (hipStream_t)stream, g_out,
                     weight, n_rows, n_out, alpha, g_h, (const int*)rows_a, (const int*)rows_b);
  return tace_check_launch("tace_radial_mlp_out_bwd_pairs_f32");
}

}  // extern "C"
