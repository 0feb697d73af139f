// Shared device helpers of the generated tensor-product translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// sum over the 64 lanes of a wavefront (cross-lane butterfly)
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// bit-reversed low 4 bits of the lane: the component index that lane holds
// after reduce16_lanes
__device__ __forceinline__ int rev4(int lane) {
  return ((lane & 1) << 3) | ((lane & 2) << 1) | ((lane & 4) >> 1) | ((lane & 8) >> 3);
}

// one butterfly level of a transposing reduction: lanes with `mask` clear keep
// the low half of v[0..2h), lanes with it set keep the high half, and each adds
// the partner lane's copy of the half it keeps
template <typename T, int H>
__device__ __forceinline__ void tr_step(T* v, int lane, int mask) {
  const bool hi = (lane & mask) != 0;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const T send = hi ? v[i] : v[i + H];
    const T keep = hi ? v[i + H] : v[i];
    v[i] = keep + __shfl_xor(send, mask, 64);
  }
}

// Sums 16 per-lane values over the 64 lanes of a wavefront with 17 shuffles.
// Lane l returns the total of component rev4(l).
template <typename T>
__device__ __forceinline__ T reduce16_lanes(T v0, T v1, T v2, T v3, T v4, T v5, T v6, T v7, T v8, T v9, T v10,
                                            T v11, T v12, T v13, T v14, T v15) {
  T v[16] = {v0, v1, v2, v3, v4, v5, v6, v7, v8, v9, v10, v11, v12, v13, v14, v15};
  const int lane = (int)threadIdx.x & 63;
  tr_step<T, 8>(v, lane, 1);
  tr_step<T, 4>(v, lane, 2);
  tr_step<T, 2>(v, lane, 4);
  tr_step<T, 1>(v, lane, 8);
  T r = v[0];
  r += __shfl_xor(r, 16, 64);
  r += __shfl_xor(r, 32, 64);
  return r;
}

// Receiver and part of this workgroup when one launch runs `nparts` part
// kernels.  Workgroups are dispatched round-robin over the 8 XCDs; the grid
// is 8 * per * nparts workgroups (per = ceil(N / 8)) and XCD k takes the
// contiguous receivers k*per .. k*per+per-1 (neighbouring receivers share
// most senders, so they hit the same L2) and, for each, its parts in
// consecutive workgroups of that XCD.  Returns -1 for padding workgroups.
__device__ __forceinline__ int tp_part_node(int n_nodes, int nparts, int* q) {
  const int per = (int)(gridDim.x >> 3) / nparts;
  const int i = (int)(blockIdx.x >> 3);
  *q = i % nparts;
  const int n = (int)(blockIdx.x & 7) * per + i / nparts;
  return n < n_nodes ? n : -1;
}

// Work of one persistent workgroup of the radial-fused tensor products: slot
// `ph` (part x channel quarter-block) and receivers [*n_begin, *n_end).  The
// grid is 8 * rpx * nph workgroups: XCD k takes the contiguous receiver ranges
// k*rpx .. k*rpx+rpx-1 of `per_range` receivers and, for each range, its nph
// slots in consecutive workgroups, so the range's senders are read into that
// XCD's L2 once for all slots.  Returns false for padding workgroups (the
// decision is uniform over the workgroup).
__device__ __forceinline__ bool rtp_slot(int n_nodes, int nph, int per_range, int* ph, int* n_begin, int* n_end) {
  const int rpx = (int)(gridDim.x >> 3) / nph;
  const int i = (int)(blockIdx.x >> 3);
  *ph = i % nph;
  const int64_t b = ((int64_t)(blockIdx.x & 7) * rpx + i / nph) * per_range;
  if (b >= n_nodes) return false;
  *n_begin = (int)b;
  *n_end = (int)(b + per_range < n_nodes ? b + per_range : n_nodes);
  return true;
}

// Cursor over the 16-edge blocks of a workgroup's receivers (receivers
// without edges have no blocks).  Uniform over the workgroup.
struct RtpCur {
  int n0, beg, end, b0;
};

// first block at receiver >= n0; false (cursor unchanged) if there is none
__device__ __forceinline__ bool rtp_seek(RtpCur& c, const int* __restrict__ rowptr, int n0, int n_end) {
  for (; n0 < n_end; ++n0) {
    const int b = rowptr[n0], e = rowptr[n0 + 1];
    if (e > b) {
      c.n0 = n0;
      c.beg = b;
      c.end = e;
      c.b0 = b;
      return true;
    }
  }
  return false;
}

// the block after c; false (cursor unchanged) at the end of the range
__device__ __forceinline__ bool rtp_next(RtpCur& c, const int* __restrict__ rowptr, int n_end) {
  if (c.b0 + 16 < c.end) {
    c.b0 += 16;
    return true;
  }
  return rtp_seek(c, rowptr, c.n0 + 1, n_end);
}

typedef float rtp_f4 __attribute__((ext_vector_type(4)));
#ifndef RTP_OCC
#define RTP_OCC __attribute__((amdgpu_waves_per_eu(2, 2)))
#endif

// A fragment of the radial-layer MFMA (v_mfma_f32_16x16x4f32, k permuted so
// that lane group g of k-step s holds k = 16 g + s): h[row][16 g .. 16 g + 15]
// of the edge in row (64 hidden features per edge), zeros for rows past the
// receiver's edges.
__device__ __forceinline__ void rtp_a_frag(const float* __restrict__ h, int ed, bool ok, int g, float* a) {
  if (ok) {
    const rtp_f4* hp = reinterpret_cast<const rtp_f4*>(h + (size_t)ed * 64 + 16 * g);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const rtp_f4 t = hp[v];
      a[4 * v] = t[0]; a[4 * v + 1] = t[1]; a[4 * v + 2] = t[2]; a[4 * v + 3] = t[3];
    }
  } else {
#pragma unroll
    for (int s = 0; s < 16; ++s) a[s] = 0.0f;
  }
}

// Sum of 16 per-lane values over each 16-lane row of the wavefront (15
// shuffles): lane l returns the row total of component rev4(l & 15).
__device__ __forceinline__ float reduce16_row(float* v) {
  const int lane = (int)threadIdx.x & 63;
  tr_step<float, 8>(v, lane, 1);
  tr_step<float, 4>(v, lane, 2);
  tr_step<float, 2>(v, lane, 4);
  tr_step<float, 1>(v, lane, 8);
  return v[0];
}
