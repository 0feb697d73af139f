// MI355X (gfx950) bf16 GEMM with float32 accumulation and output for the TECE
// SO(2) linears under the configuration's bf16 channel mixing
// (tace/models/_e3nn/archive/oam_2026_07_05.py:138-247: SO2_m0_Linear and
// SO2_m_Linear, applied per m block to the edge-frame features; the input
// gradients apply the transposed weights the same way).
//
//   out[m, n] = sum_k A[m, k] B[k, n] (+ bias[n]),   A bf16 [M, K], B bf16 [K, N]
//
// The operands are tall and skinny: M = 0.25-0.5 M edge rows per receiver
// chunk, K and N = 96..1152.  A library GEMM tiles them like square GEMMs and
// adds a bias by first copying it into the output and then accumulating with
// beta = 1.  Here:
//  * a workgroup of eight wavefronts owns RT = 16 RB rows of A (RT = 128, 64
//    or 32 by K; the A tile takes up to ~132 KB of LDS): the rows are
//    copied once into LDS (k-contiguous rows of ceil32(K) + 8 bf16, so the 16
//    rows of a fragment read fall on distinct banks) behind one barrier;
//  * the wavefronts take the output's 32-column strips in turn, each strip all
//    RT rows; B comes from a copy of the weight in MFMA fragment order (per
//    16-column block and 32-k step 512 bf16 in lane order: one coalesced
//    16-byte load per lane), one step ahead and across the end of a strip;
//  * v_mfma_f32_16x16x32_bf16 with the B fragment as the row operand, so a
//    lane holds 4 consecutive columns of one output row; the bias is added in
//    the epilogue, lanes l and l ^ 8 trade one block, and each 16-byte store
//    writes 8 whole 128-byte row segments.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tace_hip.h"

int tace_fail_msg(const char* msg);   // tace_hip.hip
int tace_check_launch(const char* what);

namespace {

typedef float gf4 __attribute__((ext_vector_type(4)));
typedef unsigned gu4 __attribute__((ext_vector_type(4)));
typedef __bf16 gbf8 __attribute__((ext_vector_type(8)));

constexpr int G_THREADS = 512, G_WAVES = G_THREADS / 64, G_SSTEP = 32 * G_WAVES;

struct GJob {
  const unsigned short* a;    // A tile row 0
  const unsigned short* bf;   // B in fragment order
  const float* bias;
  float* out;                 // out tile row 0
  int64_t ldo;
  int rows, n, nks, nb16, str;
};

// B fragments of strip c (column blocks c/16, c/16 + 1), step ks; the column
// block clamped to the last one (its outputs are not stored)
__device__ __forceinline__ void g_load_b(const GJob& J, int c, int ks, int lane, gu4 (&d)[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int jb = min((c >> 4) + j, J.nb16 - 1);
    d[j] = *(const gu4*)(J.bf + ((int64_t)jb * J.nks + ks) * 512 + 8 * lane);
  }
}

// one 32-k step of strip c: MFMAs on cur while the next step's fragments (or
// the next strip's first, cn / kn) load into nxt
template <int RB>
__device__ __forceinline__ void g_step(const unsigned short* __restrict__ As, const GJob& J, int ks, int cn, int kn,
                                       int lane, int fr, int fg, gf4 (&acc)[RB][2], const gu4 (&cur)[2],
                                       gu4 (&nxt)[2]) {
  g_load_b(J, cn, kn, lane, nxt);
  __builtin_amdgcn_sched_barrier(0);
  constexpr int PB = RB < 2 ? RB : 2;   // row blocks per A load: up to four independent accumulators
#pragma unroll
  for (int ip = 0; ip < RB / PB; ++ip) {
    gbf8 af[PB];
#pragma unroll
    for (int ii = 0; ii < PB; ++ii)
      af[ii] = *(const gbf8*)&As[(16 * (PB * ip + ii) + fr) * J.str + 32 * ks + 8 * fg];
#pragma unroll
    for (int ii = 0; ii < PB; ++ii)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[PB * ip + ii][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gbf8, cur[j]), af[ii],
                                                                       acc[PB * ip + ii][j], 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// strip c (32 columns, all RT rows); PAR: buffer of its first step; next: the
// following strip of this wavefront
template <int RB, int PAR>
__device__ __forceinline__ void g_strip(const unsigned short* __restrict__ As, const GJob& J, int c, int next,
                                        bool vst, int lane, int fr, int fg, gu4 (&b0)[2], gu4 (&b1)[2]) {
  gf4 bv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      bv[j][q] = J.bias ? J.bias[min(c + 16 * j + 4 * fg + q, J.n - 1)] : 0.f;
  }
  gf4 acc[RB][2];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = gf4{0.f, 0.f, 0.f, 0.f};
  for (int ks = 0; ks < J.nks; ks += 2) {
    const bool l0 = ks + 1 >= J.nks;
    g_step<RB>(As, J, ks, l0 ? next : c, l0 ? 0 : ks + 1, lane, fr, fg, acc, PAR ? b1 : b0, PAR ? b0 : b1);
    if (ks + 1 < J.nks) {
      const bool l1 = ks + 2 >= J.nks;
      g_step<RB>(As, J, ks + 1, l1 ? next : c, l1 ? 0 : ks + 2, lane, fr, fg, acc, PAR ? b0 : b1, PAR ? b1 : b0);
    }
  }
  // acc[i][j][q] = out[row 16 i + fr][column c + 16 j + 4 fg + q]; lanes fr and
  // fr ^ 8 trade one block: lane fr < 8 stores j = 0 of rows fr and fr + 8,
  // lane fr >= 8 j = 1 of rows fr - 8 and fr
  const bool lo = fr < 8;
  const int col = c + (lo ? 0 : 16) + 4 * fg;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const gf4 v0 = acc[i][0] + bv[0], v1 = acc[i][1] + bv[1];
    const gf4 give = lo ? v1 : v0;
    gf4 got;
#pragma unroll
    for (int q = 0; q < 4; ++q) got[q] = __shfl_xor(give[q], 8);
    const gf4 s0 = lo ? v0 : got, s1 = lo ? got : v1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 16 * i + 8 * h + (fr & 7);
      if (r >= J.rows || col >= J.n) continue;
      const gf4 v = h ? s1 : s0;
      float* dst = J.out + (int64_t)r * J.ldo + col;
      if (vst && col + 4 <= J.n) {
        __builtin_nontemporal_store(v, (gf4*)dst);   // streamed: keep L2 for B
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (col + q < J.n) dst[q] = v[q];
      }
    }
  }
}

template <int RB>
__global__ __launch_bounds__(G_THREADS) void k_so2_gemm_bf16(const unsigned short* __restrict__ a, int64_t lda,
                                                             const unsigned short* __restrict__ bfrag,
                                                             const float* __restrict__ bias, float* __restrict__ out,
                                                             int64_t ldo, int64_t M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) unsigned short As[];
  constexpr int RT = 16 * RB;
  const int64_t row0 = (int64_t)blockIdx.x * RT;
  GJob J;
  J.nks = (K + 31) >> 5;
  J.str = 32 * J.nks + 8;
  J.rows = (int)min((int64_t)RT, M - row0);
  J.n = N;
  J.nb16 = (N + 15) >> 4;
  J.a = a + row0 * lda;
  J.bf = bfrag;
  J.bias = bias;
  J.out = out + row0 * ldo;
  J.ldo = ldo;
  const int t = (int)threadIdx.x, lane = t & 63, wv = t >> 6;
  const int fr = lane & 15, fg = lane >> 4;

  // A: RT rows x K -> LDS, zeros past the rows and past K (to 32 nks); 8 bf16
  // (16 bytes) per unit
  {
    const bool avec = ((((uintptr_t)J.a) & 15) == 0) && ((lda & 7) == 0) && ((K & 7) == 0);
    const int kq = 4 * J.nks;
    for (int u = t; u < RT * kq; u += G_THREADS) {
      const int r = u / kq, kk = (u - r * kq) * 8;
      gu4 v = gu4{0u, 0u, 0u, 0u};
      if (r < J.rows) {
        const unsigned short* p = J.a + (int64_t)r * lda + kk;
        if (avec && kk + 8 <= K) {
          v = *(const gu4*)p;
        } else {
          unsigned short e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) e[q] = kk + q < K ? p[q] : (unsigned short)0;
          v = gu4{e[0] | ((unsigned)e[1] << 16), e[2] | ((unsigned)e[3] << 16), e[4] | ((unsigned)e[5] << 16),
                  e[6] | ((unsigned)e[7] << 16)};
        }
      }
      *(gu4*)&As[r * J.str + kk] = v;
    }
  }
  __syncthreads();

  const bool vst = ((ldo & 3) == 0) && ((((uintptr_t)J.out) & 15) == 0);
  // 32-column strips c = 32 (wv + G_WAVES s)
  int c = 32 * wv;
  if (c >= N) return;
  gu4 b0[2], b1[2];
  g_load_b(J, c, 0, lane, b0);
  for (; c < N; c += 2 * G_SSTEP) {
    g_strip<RB, 0>(As, J, c, c + G_SSTEP, vst, lane, fr, fg, b0, b1);
    if (c + G_SSTEP < N) {
      if (J.nks & 1) g_strip<RB, 1>(As, J, c + G_SSTEP, c + 2 * G_SSTEP, vst, lane, fr, fg, b0, b1);
      else g_strip<RB, 0>(As, J, c + G_SSTEP, c + 2 * G_SSTEP, vst, lane, fr, fg, b0, b1);
    }
  }
}

// ---- k-tiled variant: the large-k shapes ------------------------------------
// With all of a tile's k in LDS, k >= 256 leaves room for 32-64 rows only, and
// every such row tile re-reads all of B from L2.  Here a workgroup of four
// wavefronts owns a 128-row x 256-column output tile; A goes through LDS in
// 64-k stages (double-buffered, the next stage loaded into registers during
// this stage's MFMAs, one barrier per stage); wavefront w keeps the 128 x 64
// accumulator block of columns 64 w .. 64 w + 63 (32 MFMA blocks) and reads
// its B fragments from the fragment-order weight one 32-k step ahead.  Tiles
// are numbered row-tile-major and handed to the XCDs in contiguous ranges, so
// the column tiles of one row tile (same A rows) share an XCD's L2.
constexpr int KT_ROWS = 128, KT_COLS = 256, KT_KS = 64, KT_STR = KT_KS + 8;   // LDS row: 144 bytes
constexpr int KT_THREADS = 256;

struct KtJob {
  const unsigned short* a;
  const unsigned short* bf;
  const float* bias;
  float* out;
  int64_t lda, ldo;
  int rows, n, k, nks, nb16, c0;
};

// 128 x 64 of A (k0 .. k0 + 63) into registers.  AVEC (16-byte aligned rows,
// k % 64 == 0): every load unconditional and unmasked, at a clamped address --
// rows past the tile repeat its last row (their outputs are not stored); the
// prefetch past the last stage repeats it (never read).  A load under a branch, or
// one whose value a select may discard, lets the compiler move it into a
// branch, and at the join it waits for every outstanding load, the
// prefetches included.  Otherwise: zeros past the rows and past k.
template <bool AVEC>
__device__ __forceinline__ void kt_load_a(const KtJob& J, int k0, int t, gu4 (&r)[4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int u = t + KT_THREADS * q, row = u >> 3, kk = k0 + ((u & 7) << 3);
    if (AVEC) {
      r[q] = *(const gu4*)(J.a + (int64_t)min(row, J.rows - 1) * J.lda + min(kk, J.k - 8));
    } else {
      gu4 v = gu4{0u, 0u, 0u, 0u};
      if (row < J.rows) {
        const unsigned short* p = J.a + (int64_t)row * J.lda + kk;
        unsigned short e[8];
#pragma unroll
        for (int z = 0; z < 8; ++z) e[z] = kk + z < J.k ? p[z] : (unsigned short)0;
        v = gu4{e[0] | ((unsigned)e[1] << 16), e[2] | ((unsigned)e[3] << 16), e[4] | ((unsigned)e[5] << 16),
                e[6] | ((unsigned)e[7] << 16)};
      }
      r[q] = v;
    }
  }
}

// AVEC with this thread's four row pointers made once (row clamped, k offset
// of its 8-element run included): a stage's load is pointer + k0
__device__ __forceinline__ void kt_load_a_p(const unsigned short* const (&ap)[4], int k0, gu4 (&r)[4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) r[q] = *(const gu4*)(ap[q] + k0);
}

__device__ __forceinline__ void kt_store_a(unsigned short* __restrict__ As, int t, const gu4 (&r)[4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int u = t + KT_THREADS * q;
    *(gu4*)&As[(u >> 3) * KT_STR + ((u & 7) << 3)] = r[q];
  }
}

// B fragments of the wavefront's four 16-column blocks at 32-k step ks (the
// column block clamped to the last one: its outputs are not stored)
__device__ __forceinline__ void kt_load_b(const KtJob& J, int cw, int ks, int lane, gu4 (&d)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int jb = min((cw >> 4) + j, J.nb16 - 1);
    d[j] = *(const gu4*)(J.bf + ((int64_t)jb * J.nks + ks) * 512 + 8 * lane);
  }
}

template <bool AVEC>
__global__ __launch_bounds__(KT_THREADS, 2) void k_so2_gemm_kt(const unsigned short* __restrict__ a, int64_t lda,
                                                             const unsigned short* __restrict__ bfrag,
                                                             const float* __restrict__ bias, float* __restrict__ out,
                                                             int64_t ldo, int64_t M, int N, int K, int n_rt, int n_ct,
                                                             int per) {
  __shared__ __attribute__((aligned(16))) unsigned short As[2][KT_ROWS * KT_STR];
  const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (tile >= n_rt * n_ct) return;
  const int rt = tile / n_ct, ct = tile - rt * n_ct;
  const int64_t row0 = (int64_t)rt * KT_ROWS;
  KtJob J;
  J.a = a + row0 * lda;
  J.bf = bfrag;
  J.bias = bias;
  J.out = out + row0 * ldo;
  J.lda = lda;
  J.ldo = ldo;
  J.rows = (int)min((int64_t)KT_ROWS, M - row0);
  J.n = N;
  J.k = K;
  J.nks = (K + 31) >> 5;
  J.nb16 = (N + 15) >> 4;
  J.c0 = ct * KT_COLS;
  const int t = (int)threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int cw = J.c0 + 64 * wv;          // the wavefront's first column
  const bool has_cols = cw < N;           // otherwise it only stages A
  const int n_st = (J.nks + 1) >> 1;      // 64-k stages

  gf4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = gf4{0.f, 0.f, 0.f, 0.f};

  const unsigned short* ap[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int u = t + KT_THREADS * q;
    ap[q] = J.a + (int64_t)min(u >> 3, J.rows - 1) * J.lda + ((u & 7) << 3);
  }
  auto load_a = [&](int k0, gu4 (&r)[4]) {
    if constexpr (AVEC) kt_load_a_p(ap, k0, r);
    else kt_load_a<AVEC>(J, k0, t, r);
  };
  gu4 ra[4];
  load_a(0, ra);
  kt_store_a(As[0], t, ra);
  __syncthreads();
  if (has_cols) {
    gu4 b0[4], b1[4];
    kt_load_b(J, cw, 0, lane, b0);
    for (int st = 0; st < n_st; ++st) {
      const unsigned short* __restrict__ Ab = As[st & 1];
      const int ks0 = 2 * st;
      // every load unconditional: past the last stage / step they repeat it
      load_a(min(st + 1, n_st - 1) * KT_KS, ra);
      kt_load_b(J, cw, min(ks0 + 1, J.nks - 1), lane, b1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const gbf8 af = *(const gbf8*)&Ab[(16 * i + fr) * KT_STR + 8 * fg];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gbf8, b0[j]), af, acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      kt_load_b(J, cw, min(ks0 + 2, J.nks - 1), lane, b0);
      __builtin_amdgcn_sched_barrier(0);
      if (AVEC || ks0 + 1 < J.nks) {   // AVEC: k % 64 == 0, every stage has both steps
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const gbf8 af = *(const gbf8*)&Ab[(16 * i + fr) * KT_STR + 32 + 8 * fg];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gbf8, b1[j]), af, acc[i][j], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      kt_store_a(As[(st + 1) & 1], t, ra);
      __syncthreads();
    }
  } else {
    for (int st = 0; st < n_st; ++st) {
      load_a(min(st + 1, n_st - 1) * KT_KS, ra);
      kt_store_a(As[(st + 1) & 1], t, ra);
      __syncthreads();
    }
  }
  if (!has_cols) return;

  // epilogue: acc[i][j][q] = out[row 16 i + fr][column cw + 16 j + 4 fg + q];
  // per pair of column blocks (j, j + 1) lanes fr and fr ^ 8 trade one block
  // so that each 16-byte store writes whole 128-byte row segments
  const bool lo = fr < 8;
  const bool vst = ((J.ldo & 3) == 0) && ((((uintptr_t)J.out) & 15) == 0);
#pragma unroll
  for (int jp = 0; jp < 2; ++jp) {
    const int cb = cw + 32 * jp;
    gf4 bv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bv[j][q] = J.bias ? J.bias[min(cb + 16 * j + 4 * fg + q, N - 1)] : 0.f;
    const int col = cb + (lo ? 0 : 16) + 4 * fg;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const gf4 v0 = acc[i][2 * jp] + bv[0], v1 = acc[i][2 * jp + 1] + bv[1];
      const gf4 give = lo ? v1 : v0;
      gf4 got;
#pragma unroll
      for (int q = 0; q < 4; ++q) got[q] = __shfl_xor(give[q], 8);
      const gf4 s0 = lo ? v0 : got, s1 = lo ? got : v1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 16 * i + 8 * h + (fr & 7);
        if (r >= J.rows || col >= N) continue;
        const gf4 v = h ? s1 : s0;
        float* dst = J.out + (int64_t)r * J.ldo + col;
        if (vst && col + 4 <= N) {
          __builtin_nontemporal_store(v, (gf4*)dst);   // streamed: keep L2 for A and B
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (col + q < N) dst[q] = v[q];
        }
      }
    }
  }
}

}  // namespace

extern "C" int tace_so2_gemm_bf16_kt(const uint16_t* a, int64_t lda, const uint16_t* b_frag, const float* bias,
                                     float* out, int64_t ldo, int64_t m, int32_t n, int32_t k, void* stream) {
  if (m < 0 || n <= 0 || k <= 0 || k > 65536 || lda < k || ldo < n)
    return tace_fail_msg("tace_so2_gemm_bf16_kt: bad sizes (0 < n, 0 < k <= 65536, lda >= k, ldo >= n)");
  if (m == 0) return 0;
  if (!a || !b_frag || !out) return tace_fail_msg("tace_so2_gemm_bf16_kt: null pointer");
  if ((((uintptr_t)b_frag) & 15) != 0)
    return tace_fail_msg("tace_so2_gemm_bf16_kt: the fragment-order weight must be 16-byte aligned");
  const int64_t n_rt = (m + KT_ROWS - 1) / KT_ROWS, n_ct = (n + KT_COLS - 1) / KT_COLS;
  if (n_rt * n_ct > 0x7fffffffll / 2) return tace_fail_msg("tace_so2_gemm_bf16_kt: too many rows");
  const int64_t per = (n_rt * n_ct + 7) / 8;
  const bool avec = ((((uintptr_t)a) & 15) == 0) && ((lda & 7) == 0) && ((k & 63) == 0);
  if (avec)
    hipLaunchKernelGGL(k_so2_gemm_kt<true>, dim3((unsigned)(8 * per)), dim3(KT_THREADS), 0, (hipStream_t)stream,
                       (const unsigned short*)a, lda, (const unsigned short*)b_frag, bias, out, ldo, m, (int)n, (int)k,
                       (int)n_rt, (int)n_ct, (int)per);
  else
    hipLaunchKernelGGL(k_so2_gemm_kt<false>, dim3((unsigned)(8 * per)), dim3(KT_THREADS), 0, (hipStream_t)stream,
                       (const unsigned short*)a, lda, (const unsigned short*)b_frag, bias, out, ldo, m, (int)n, (int)k,
                       (int)n_rt, (int)n_ct, (int)per);
  return tace_check_launch("tace_so2_gemm_bf16_kt");
}

extern "C" int tace_so2_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b_frag, const float* bias, float* out,
                                  int64_t ldo, int64_t m, int32_t n, int32_t k, void* stream) {
  if (m < 0 || n <= 0 || k <= 0 || k > 2048 || lda < k || ldo < n)
    return tace_fail_msg("tace_so2_gemm_bf16: bad sizes (0 < n, 0 < k <= 2048, lda >= k, ldo >= n)");
  if (m == 0) return 0;
  if (!a || !b_frag || !out) return tace_fail_msg("tace_so2_gemm_bf16: null pointer");
  if ((((uintptr_t)b_frag) & 15) != 0)
    return tace_fail_msg("tace_so2_gemm_bf16: the fragment-order weight must be 16-byte aligned");
  const int nks = (k + 31) / 32;
  hipStream_t s = (hipStream_t)stream;
#define SO2_G(RB)                                                                                                    \
  do {                                                                                                               \
    const int64_t tiles = (m + 16 * (RB) - 1) / (16 * (RB));                                                          \
    if (tiles > 0x7fffffff) return tace_fail_msg("tace_so2_gemm_bf16: too many rows");                              \
    const size_t lds = (size_t)16 * (RB) * (32 * nks + 8) * 2;                                                        \
    if (lds > 65536 &&                                                                                               \
        hipFuncSetAttribute((const void*)k_so2_gemm_bf16<RB>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)   \
            != hipSuccess)                                                                                           \
      return tace_fail_msg("tace_so2_gemm_bf16: cannot reserve the LDS tile");                                       \
    hipLaunchKernelGGL(k_so2_gemm_bf16<RB>, dim3((unsigned)tiles), dim3(G_THREADS), lds, s,                         \
                       (const unsigned short*)a, lda, (const unsigned short*)b_frag, bias, out, ldo, m, (int)n,     \
                       (int)k);                                                                                      \
  } while (0)
  // rows per workgroup by k: the A tile takes at most ~132 KB of LDS
  if (k <= 376) SO2_G(8);
  else if (k <= 1016) SO2_G(4);
  else SO2_G(2);
#undef SO2_G
  return tace_check_launch("tace_so2_gemm_bf16");
}
