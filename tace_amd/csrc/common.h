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
