/* C ABI of libtace_hip.so -- MI355X (gfx950) kernels of the TACE/TECE
 * energy-and-force path.
 *
 * Conventions
 *   - Every pointer argument except `cell`/`pbc` (host arrays) is a device
 *     pointer allocated by the caller (PyTorch on ROCm); the library never
 *     allocates device memory and never holds a pointer after returning.
 *   - `stream` is a hipStream_t; launches are asynchronous on it, nothing
 *     synchronises the host.
 *   - Return value: 0 on success, < 0 on error; tace_last_error() returns a
 *     thread-local message for the last failure.
 *   - dtype: TACE_F32 or TACE_F64; all float arrays of one call share it (five TECE
 *     functions also take TACE_F32_BF16, see below).
 *   - Node features use e3nn's mul_ir layout: irrep blocks concatenated,
 *     each block [channels, 2l+1] row-major.
 *
 * Reference interfaces replaced (xvzemin/tace, paths relative to its root):
 *   tace_edge_tp_fwd / _bwd   O3ScatterTensorProduct.forward(x, y, w, edge_index)
 *                             tace/models/_e3nn/fused.py:259-271 (the `fused_tp`
 *                             plug-in slot filled at fused.py:218-257; same
 *                             contract as oeq/_tp_scatter.py:53-93)
 *   tace_uuu_fwd / _bwd       uuuTensorProduct.forward(x, y)  fused.py:90-95
 *                             (plug-in slot fused.py:61-71)
 *   tace_edge_basis_fwd/_bwd  RadialBasis.forward (radial.py:974-993: j0 Bessel
 *                             43-84 x C2PolynomialCutoff 437-472) and
 *                             SphericalHarmonics.forward (angular.py:288-315)
 *                             as called at representation.py:305-324
 *   tace_edge_vec_fwd/_bwd    edge vectors of TensorModel.prepare_graph
 *                             (models/adapter.py:334-340) and their position gradient
 *   tace_nl_*                 get_neighborhood (dataset/neighbour_list.py:195-298)
 *   tace_edge_wigner_*, tace_tece_*, tace_graph_softmax_*
 *                             TECE convolution pieces, see their section below
 */
#ifndef TACE_HIP_H
#define TACE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TACE_HIP_ABI_VERSION 32
#define TACE_MAX_CHANNELS 512
#define TACE_F32 0
#define TACE_F64 1
/* float32 arithmetic and inputs; the outputs that feed the TECE SO(2)-linear
 * GEMMs stored as bfloat16 (round to nearest even).  Accepted by
 * tace_edge_rotate_in_fwd (m_src, m_dst, m_w), tace_tece_edge_ace_fwd (o*),
 * tace_tece_edge_ace_bwd (g_y*), tace_tece_score_bwd (g_q, g_k) and
 * tace_tece_rotate_out_bwd (g_m); every other output stays float32. */
#define TACE_F32_BF16 2

const char* tace_last_error(void);
int tace_abi_version(void);
/* Measurement hook (no counterpart in the reference; for profilers that
 * bracket an entry point with events): the next tace_edge_tp_bwd,
 * tace_edge_tp_bwd_rows or tace_edge_tp_bwd_noalloc call made on this host
 * thread records `hip_event` (a hipEvent_t) on its stream right after its
 * product kernel, before the grad_y and grad_x sums, and the mark is then
 * cleared.  NULL clears a pending mark.  Returns 0. */
int tace_mark_phase_event(void* hip_event);

/* ---- tensor-product variants -------------------------------------------
 * A variant is keyed by "kind|in1 ls|in2 ls|out ls", e.g.
 * "uvu|0,1,2,3|0,1,2,3|0,1,2,3"; paths follow generate_paths
 * (tace/models/_e3nn/paths.py:30-71).  d1/d2/dout are per-channel widths. */
int tace_tp_num_variants(void);
const char* tace_tp_variant_key(int vid);
int tace_tp_find(const char* key);
int tace_tp_dims(int vid, int32_t* npath, int32_t* d1, int32_t* d2, int32_t* dout);

/* Operand layouts.  e3nn (0): node features in e3nn's mul_ir layout.
 * Group-major: the runs of equal-l blocks that Irreps.simplify() merges form
 * groups g; group g of the whole batch is one row-major [N, 2l+1, count_g*C]
 * matrix at element offset N*C*goff_g (goff_g = per-channel offset of the
 * group) -- the operand layout of the channel-mixing GEMMs that consume it. */
#define TACE_LAYOUT_IN1_GROUPED 1
#define TACE_LAYOUT_OUT_GROUPED 2
#define TACE_LAYOUT_IN2_GROUPED 4 /* uuu only: x2 / g2 */

/* out[n] = sum_{e: dst(e)=n} TP(x[src(e)], y[e], w[e])  -- uvu, mul2 = 1.
 * Edges are visited in receiver-CSR order: rowptr[n_nodes+1] over the sorted
 * edge list, eid[k] the edge id of sorted slot k (NULL = identity), src[e] the
 * sender of edge id e.  x [N, C*d1], y [E, d2], w [E, C*npath], out [N, C*dout];
 * 1 <= C <= TACE_MAX_CHANNELS.  node_map[N] (NULL = identity) gives the row
 * of node n in x / out / gout / gx: the features may be stored in another node
 * order (e.g. grouped by species) than the one the edges index.  layout: any
 * combination of TACE_LAYOUT_IN1_GROUPED (x, gx) and TACE_LAYOUT_OUT_GROUPED
 * (out, gout). */
int tace_edge_tp_fwd(int vid, int dtype, const void* x, const void* y, const void* w, const int32_t* rowptr,
                     const int32_t* eid, const int32_t* src, const int32_t* node_map, int64_t n_nodes, int64_t n_edges,
                     int32_t channels, int32_t layout, void* out, void* stream);
/* Gradients of sum(gout * out): gy [E, d2], gw [E, C*npath]; gx [N, C*d1]
 * (NULL to skip).  All outputs are fully overwritten, no atomics: the
 * per-edge grad_x contributions go to `workspace` (one row per
 * receiver-sorted slot) and are summed per sender through the sender CSR:
 * s_rowptr[N+1], s_slot[E] = receiver-sorted slots grouped by sender.  gy is
 * summed over channels and kernel parts in a fixed order.  `workspace` holds
 * at least tace_edge_tp_workspace_elems(vid, E, C, gx != NULL) elements. */
int64_t tace_edge_tp_workspace_elems(int vid, int64_t n_edges, int32_t channels, int32_t need_gx);
int tace_edge_tp_bwd(int vid, int dtype, const void* x, const void* y, const void* w, const void* gout,
                     const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                     int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout, const int32_t* s_rowptr, const int32_t* s_slot,
                     void* workspace, int64_t workspace_elems, void* gx, void* gy, void* gw, void* stream);

/* The same products with the weight rows indexed through w_rows (int32 [E],
 * by edge id; NULL = the edge id itself): edge e uses w[w_rows[e]] and
 * w has as many rows as w_rows names.  The two directions of an edge (i -> j
 * with shift S, j -> i with -S) have one length, so the radial MLP's weights
 * (tace/models/_e3nn/inter.py:166-183) are the same for both and can be made
 * once per pair (tace_edge_pairs).  gw stays per edge: [E, C*npath]. */
int tace_edge_tp_fwd_rows(int vid, int dtype, const void* x, const void* y, const void* w, const int32_t* rowptr,
                          const int32_t* eid, const int32_t* src, const int32_t* node_map, const int32_t* w_rows,
                          int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout, void* out,
                          void* stream);
int tace_edge_tp_bwd_rows(int vid, int dtype, const void* x, const void* y, const void* w, const void* gout,
                          const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                          const int32_t* w_rows, int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                          const int32_t* s_rowptr, const int32_t* s_slot, void* workspace, int64_t workspace_elems,
                          void* gx, void* gy, void* gw, void* stream);

/* tace_edge_tp_bwd for callers that cannot allocate device memory (code under
 * HIP graph capture, tight MD/serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference: it exists for those callers.
 * Same arguments, results and rules as tace_edge_tp_bwd, without the
 * workspace: the per-slot grad_x rows and grad_y partials go to a library-owned
 * device array of TACE_NOALLOC_SCRATCH_BYTES per GPU (held until the process
 * ends; its address is looked up once per device on the first call with that
 * device current).  A call whose workspace (tace_edge_tp_workspace_elems x
 * element size) exceeds it fails with an error before any device work.  The
 * call allocates nothing.  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (e.g. on two streams, or from two
 * threads) race and give wrong results -- serialise them.  Devices with an
 * index >= TACE_NOALLOC_MAX_DEVICES are refused. */
#define TACE_NOALLOC_SCRATCH_BYTES (64ll << 20)
#define TACE_NOALLOC_MAX_DEVICES 64
int tace_edge_tp_bwd_noalloc(int vid, int dtype, const void* x, const void* y, const void* w, const void* gout,
                             const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                             int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                             const int32_t* s_rowptr, const int32_t* s_slot, void* gx, void* gy, void* gw,
                             void* stream);

/* The same product with the radial MLP's last layer folded in (float32):
 * w[e, p*C + u] = alpha * sum_k h[e, k] w_last[k, p*C + u] -- the last
 * mlpLinear of the radial network (tace/models/mlp.py:136-191) feeding the
 * weights of the edge product (tace/models/_e3nn/fused.py:218-271) -- is made
 * inside the kernel on MFMA and never stored.  h [E, 64] (the last hidden
 * activations, 16-byte aligned), w_last [64, C*npath]; C a multiple of 64;
 * slot_rows: n_edges int32 of scratch (the sender's feature row of every
 * receiver-sorted slot, filled by the call); the other arguments and
 * layouts as in tace_edge_tp_fwd.  out equals
 * tace_edge_tp_fwd with w from that layer, up to the order in which each
 * receiver's edges are summed (fixed: results repeat bit for bit). */
int tace_edge_rtp_fwd(int vid, const float* x, const float* y, const float* h, const float* w_last, float alpha,
                      const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* node_map,
                      int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout, int32_t* slot_rows,
                      float* out, void* stream);
/* Gradients of sum(gout * out) as in tace_edge_tp_bwd: gy [E, d2], gw [E,
 * C*npath] = grad of the per-edge weights w (the caller forms the h gradient
 * as alpha * gw @ w_last^T), gx [N, C*d1] (NULL to skip); the weights are
 * recomputed on MFMA.  `workspace` holds at least
 * tace_edge_rtp_workspace_elems(vid, E, C, gx != NULL) floats. */
int64_t tace_edge_rtp_workspace_elems(int vid, int64_t n_edges, int32_t channels, int32_t need_gx);
int tace_edge_rtp_bwd(int vid, const float* x, const float* y, const float* h, const float* w_last, float alpha,
                      const float* gout, const int32_t* rowptr, const int32_t* eid, const int32_t* src,
                      const int32_t* node_map, int64_t n_nodes, int64_t n_edges, int32_t channels, int32_t layout,
                      const int32_t* s_rowptr, const int32_t* s_slot, int32_t* slot_rows, float* workspace,
                      int64_t workspace_elems, float* gx, float* gy, float* gw, void* stream);

/* out[n] = uuu(x1[n], x2[n]); x1 [N, C*d1], x2 [N, C*d2], out [N, C*dout].
 * Weighted variants (the bilinear-gate products, second operand = hidden
 * irreps + one 0e block) take w [N, npath*C], which scales path p of channel
 * u by w[n, p*C + u] -- the trainable product of _e3nn/prod.py:126-147 /
 * fused.py:17-95 -- and their backward also writes gw [N, npath*C]; all
 * other variants take w = NULL.  A mismatch is an error.
 * layout flags select the group-major layout for x1 (and g1), out (and
 * gout) and x2 (and g2).  Accepted: 0, OUT_GROUPED, IN1_GROUPED|OUT_GROUPED,
 * IN1_GROUPED|OUT_GROUPED|IN2_GROUPED. */
int tace_uuu_fwd(int vid, int dtype, const void* x1, const void* x2, const void* w, int64_t n_nodes, int32_t channels,
                 int32_t layout, void* out, void* stream);
/* Gradients g1 [N, C*d1], g2 [N, C*d2] (and gw for weighted variants) of
 * sum(gout * out).  Variants with many x1 blocks run their backward in parts
 * (one per group of x1 blocks) whose g2 partials go to `workspace` (at least
 * tace_uuu_workspace_elems(vid, N, C, accumulate) elements; 0 for one part
 * without accumulate bit 1, then workspace may be NULL) and are summed in a
 * fixed order.  accumulate bit 0 adds grad_x1 to what g1 holds, bit 1 adds
 * grad_x2 to what g2 holds (instead of overwriting them): the gradient sums of
 * a tensor that other operators read too.  An accumulated gradient is staged
 * in the workspace and added after the product kernel, grad_x1 first, so g1
 * and g2 may be the same array when both bits are set and x1 and x2 are in
 * one layout (the product of a tensor with itself). */
int64_t tace_uuu_workspace_elems(int vid, int64_t n_nodes, int32_t channels, int32_t accumulate);
int tace_uuu_bwd(int vid, int dtype, const void* x1, const void* x2, const void* w, const void* gout, int64_t n_nodes,
                 int32_t channels, int32_t layout, void* g1, void* g2, void* gw, void* workspace,
                 int64_t workspace_elems, int32_t accumulate, void* stream);

/* ---- edge featurisation --------------------------------------------------
 * vec [E, 3] edge vectors; r = |vec| + 1e-9;
 * radial[E, nb] = prefactor * sin(bessel_w[n] r) / r * f(r/cutoff) * [r < cutoff]
 * sh[E, (lmax+1)^2] = component-normalised real SH of vec / r (e3nn order). */
int tace_edge_basis_fwd(int dtype, const void* vec, int64_t n_edges, int32_t num_basis, const void* bessel_w,
                        double prefactor, double cutoff, int32_t poly_p, int32_t lmax, void* radial, void* sh,
                        void* stream);
int tace_edge_basis_bwd(int dtype, const void* vec, const void* g_radial, const void* g_sh, int64_t n_edges,
                        int32_t num_basis, const void* bessel_w, double prefactor, double cutoff, int32_t poly_p,
                        int32_t lmax, void* g_vec, void* stream);

/* ---- edge vectors --------------------------------------------------------
 * vec[e] = pos[dst[e]] - pos[src[e]] + shifts[e] . lattice[edge_graph[e]]
 * (edge_graph NULL = graph 0).  The backward gives
 * g_pos[n] = sum_{e: dst=n} g_vec[e] - sum_{e: src=n} g_vec[e] in the fixed
 * order of the receiver CSR (rowptr, eid) and the sender CSR (s_rowptr,
 * s_slot over receiver-sorted slots); no atomics. */
int tace_edge_vec_fwd(int dtype, const void* pos, const void* lattice, const int32_t* src, const int32_t* dst,
                      const void* shifts, const int32_t* edge_graph, int64_t n_edges, void* vec, void* stream);
int tace_edge_vec_bwd(int dtype, const void* g_vec, const int32_t* rowptr, const int32_t* eid,
                      const int32_t* s_rowptr, const int32_t* s_slot, int64_t n_nodes, void* g_pos, void* stream);

/* ---- radial MLP hidden layers (tace/models/mlp.py:136-191): h_0 = radial
 * [E, n_in], h_l = silu(h_(l-1) W_l) for l = 1..n_layers, every hidden width
 * TACE_MLP_WIDTH; the last (wide, linear) layer of the MLP is a GEMM left to
 * the caller.  weights: the n_layers matrices packed row-major
 * [n_in x 64 | 64 x 64 | ...] with their scale folded in.  Output: h [E, 64]
 * (the last hidden activations, row-major).  float32 runs on fp32 MFMA,
 * float64 per edge on the vector ALUs.
 *   tace_radial_mlp_bwd: g_radial [E, n_in] from g_h [E, 64], recomputing the
 *   pre-activations from radial (nothing is saved between the two; weights
 *   are constants: no weight gradient). */
#define TACE_MLP_WIDTH 64
#define TACE_MLP_MAX_IN 32
#define TACE_MLP_MAX_LAYERS 4
int tace_radial_mlp_fwd(int dtype, const void* radial, int64_t n_edges, int32_t n_in, int32_t n_layers,
                        const void* weights, void* h, void* stream);
int tace_radial_mlp_bwd(int dtype, const void* radial, const void* g_h, int64_t n_edges, int32_t n_in,
                        int32_t n_layers, const void* weights, void* g_radial, void* stream);
/* the last (linear) layer in float32: out [E, n_out] = alpha h [E, 64] @
 * weight [64, n_out] (row-major; h 16-byte aligned), on the bf16 MFMA with
 * both operands split exactly into three bf16 terms (float32 rounding).
 *   tace_radial_mlp_out_bwd_f32: its input gradient (the backward of the
 *   last Linear of mlp.py:136-191), g_h [E, 64] = alpha g_out [E, n_out] @
 *   weight^T, the same way (g_out and weight 16-byte aligned when n_out is a
 *   multiple of 4; weights are constants: no weight gradient). */
int tace_radial_mlp_out_f32(const float* h, const float* weight, int64_t n_edges, int32_t n_out, float alpha,
                            float* out, void* stream);
int tace_radial_mlp_out_bwd_f32(const float* g_out, const float* weight, int64_t n_edges, int32_t n_out, float alpha,
                                float* g_h, void* stream);
/* the same for weight rows shared by edge pairs: g_h [n_rows, 64] = alpha
 * (g_out[rows_a[r]] + g_out[rows_b[r]]) @ weight^T, the sum in float32
 * (rows_b[r] < 0: g_out[rows_a[r]] alone); g_out [E, n_out] per edge. */
int tace_radial_mlp_out_bwd_pairs_f32(const float* g_out, const int32_t* rows_a, const int32_t* rows_b,
                                      int64_t n_rows, int32_t n_out, float alpha, const float* weight, float* g_h,
                                      void* stream);

/* ---- per-species (element) linears
 * tace_seg_linear replaces the per-element o3.Linear of e3nnElementLinear
 * (tace/models/linear.py:377-482) on species-sorted, group-major node
 * features: every output block, species and instruction of one linear (or of
 * its input gradient) in one launch.  The work is a table of n_tiles output
 * tiles of tile_rows x tile_cols elements (128 x 128: float32 on MFMA;
 * 64 x 64: float32 or float64 on FMA), each inside one output block and one
 * species' rows:
 *   tiles    int64 [n_tiles, 8]: out_base (element offset of the tile's first
 *            row in y), rows (1..tile_rows), n (block width = row stride), c0 (first
 *            column), bias_off (offset into bias, -1 none), cb, ce (its
 *            contributions [cb, ce)), unused;
 *   contribs int64 [*, 4]: x_base (offset of the tile's first row in x), k
 *            (input block width = row stride), w_off (offset of the weight
 *            matrix in w), trans (0: W is [k, n] row-major; 1: W is [n, k]
 *            row-major and W^T is applied -- the input gradient);
 *   scales   double [*]: the contribution's path weight.
 * y[tile] = addend[tile] + alpha (sum_c scale_c x_c[rows] @ W_c +
 * bias[bias_off + cols]), addend optional (null: no term) and either y itself
 * (y += ..., the gradient sums of a tensor read by several linears) or an
 * array of y's size that does not overlap y.  The entry points below take
 * addend the same way; their MFMA kernels (tace_seg_linear_presplit_frag and
 * tace_seg_linear_presplit_ks) start each sum from addend / alpha, so there
 * the result equals the formula up to float32 rounding and alpha must not be
 * 0 when addend is given.  Every tile element is written; tiles must not
 * overlap.  The tables live in
 * device memory and are trusted: the host builds them from the layout
 * (tace_amd.ops.SegLinearPlan) and checks every offset against the array
 * sizes before upload. */
int tace_seg_linear(int dtype, int32_t tile_rows, int32_t tile_cols, const void* x, void* y, const void* addend,
                    const void* w, const void* bias, const int64_t* tiles, int64_t n_tiles, const int64_t* contribs,
                    const double* scales, double alpha, void* stream);
/* The float32 128 x 128 case with the weights split ahead of time (they are
 * constants at inference; the same e3nnElementLinear forward and input
 * gradient, linear.py:377-482).
 *   tace_bf16x3_split_blocks writes, for n_blocks weight blocks (int64 [n, 6]:
 *   src_off, cols, k, transpose, dst_off, layout; double scales[n]), the three
 *   bf16 terms of scale * B (the exact split of float32 into three bf16, round
 *   to nearest even), with B[kk][c] = w[src_off + kk cols + c] (transpose = 1:
 *   the forward's W [k, n]) or w[src_off + c k + kk] (transpose = 0: W [n, k]
 *   applied transposed, the input gradient) and zeros past k and cols:
 *     layout 0: term p into planes[p * plane_stride + dst_off + c k_pad + kk]
 *               for column c < cols and kk < k_pad = ceil8(k);
 *     layout 1 (MFMA fragment order, for tace_seg_linear_presplit_ks and
 *               tace_seg_linear_presplit_frag): one
 *               buffer, per 16-column block cb and 32-k step s (nks =
 *               ceil(k / 32) steps per column block, ceil16(cols) columns)
 *               the three terms as runs of 512: element (c, kk) of term p at
 *               planes[dst_off + ((cb nks + s) 3 + p) 512 + (((kk % 32) / 8)
 *               16 + c % 16) 8 + kk % 8], cb = c / 16, s = kk / 32;
 *               plane_stride is unused.
 *   tace_seg_linear_presplit then runs the tile table of tace_seg_linear with
 *   each contribution's w_off pointing at its block in the planes (16-byte
 *   aligned, plane_stride a multiple of 8); trans and the scales are unused
 *   (folded into the planes).  The products and their order are those of
 *   tace_seg_linear's float32 128 x 128 kernel, so the outputs are the same
 *   bits. */
int tace_bf16x3_split_blocks(const float* w, const int64_t* blocks, const double* scales, int64_t n_blocks,
                             uint16_t* planes, int64_t plane_stride, void* stream);
int tace_seg_linear_presplit(const float* x, float* y, const float* addend, const uint16_t* w_planes,
                             int64_t plane_stride, const float* bias, const int64_t* tiles, int64_t n_tiles, const int64_t* contribs,
                             double alpha, void* stream);
/* The same linears' tiles with one contribution of k <= 256 (the input
 * gradients of the product-basis contractions, linear.py:377-482, and any
 * block with no contribution), as n_tasks row tiles of up to task_rows rows,
 * each over a column range, with the weights split in MFMA fragment order
 * (tace_bf16x3_split_blocks layout 1).  task_rows is 128 (every task's k <=
 * 128) or 64 (k <= 256): tace_seg_linear_ks_rows(k) gives the height for k
 * (0: not supported); one call takes tasks of one height.  A task whose k
 * exceeds its height's limit (128 for 128-row tasks, 256 for 64-row tasks)
 * gets NaN in every output of its tile:
 *   tasks int64 [n_tasks, 10]: out_base (offset of the tile's row 0, column 0
 *         in y), rows (1..task_rows), n (block width = row stride of y), cb, ce (its
 *         columns [cb, ce), ce <= n), bias_off (-1 none), x_base (offset of
 *         the tile's row 0 in x), k (0..256, the row stride of x; 0: no
 *         contribution), w_off (the block's offset in w_frag), unused.
 * y[tile] = addend[tile] + alpha (x[rows, :k] @ B + bias[bias_off + cols]), the same bits as
 * tace_seg_linear_presplit gives for the same tile.  Trusted tables, checked
 * by the host (tace_amd.ops.SegLinearPlan). */
int32_t tace_seg_linear_ks_rows(int32_t k);
/* The tile table of tace_seg_linear_presplit (same tiles and contributions,
 * any k) with each contribution's w_off pointing at its block in weights
 * split in MFMA fragment order (tace_bf16x3_split_blocks layout 1, 16-byte
 * aligned): B is read from there one 32-k step ahead instead of being staged
 * in LDS.  aligned != 0 promises that every contribution's x offset and k are
 * multiples of 4 (16-byte rows of x; with x 16-byte aligned the kernel then
 * loads A without per-element tails).  The same bits as
 * tace_seg_linear_presplit for the same tiles. */
int tace_seg_linear_presplit_frag(const float* x, float* y, const float* addend, const uint16_t* w_frag,
                                  const float* bias,
                                  const int64_t* tiles, int64_t n_tiles, const int64_t* contribs, int32_t aligned,
                                  double alpha, void* stream);
int tace_seg_linear_presplit_ks(const float* x, float* y, const float* addend, const uint16_t* w_frag,
                                const float* bias,
                                const int64_t* tasks, int64_t n_tasks, int32_t task_rows, double alpha, void* stream);
/* tace_seg_linear_presplit_frag with k split over `splits` (2..64)
 * workgroups per tile, for launches with too few tiles to fill the GPU (the
 * small systems' per-species linears, linear.py:377-482): every tile has at
 * most one contribution (a tile with more gets NaN in every output); work
 * item tile * splits + s sums 32-k steps [s nks / splits, (s + 1) nks /
 * splits) of it into partials[(tile splits + s) 16384 ..] (a 128 x 128 tile,
 * row stride 128; partial_elems >= n_tiles splits 16384 floats, 16-byte
 * aligned, no other use during the call), and a second kernel writes y[tile]
 * = alpha (addend / alpha + partial_0 + ... + partial_{splits-1} + bias),
 * the partials in split order: every run gives the same bits, which differ
 * from the unsplit kernel's by float32 summation order. */
int tace_seg_linear_presplit_frag_split(const float* x, float* y, const float* addend, const uint16_t* w_frag,
                                        const float* bias, const int64_t* tiles, int64_t n_tiles,
                                        const int64_t* contribs, int32_t aligned, int32_t splits, float* partials,
                                        int64_t partial_elems, double alpha, void* stream);

/* ---- TECE radial-rotary edge attention (config 5)
 * K = (lmax+1)^2 edge-frame components with mmax = lmax; the "m layout"
 * orders them m = 0 (l = 0..lmax), then per m = 1..lmax the +m rows and the
 * -m rows (tace/models/o2/wigner.py:38-66).
 * Edge features with ch channels are passed in the SO(2) block layout, as an
 * array of lmax+1 block pointers: block 0 is [E, (lmax+1) ch] (the m = 0
 * rows), block m is [2E, (lmax+1-m) ch] with row 2e the +m rows and row 2e+1
 * the -m rows of edge e -- each block is one SO(2)-linear GEMM operand.
 *   tace_edge_wigner_fwd/_bwd   WignerD.get_wigner (o2/wigner.py:231-239) with
 *                               init_edge_rot_mat_quaternion (o2/rotation_matrix.py:74-88):
 *                               wigner [E, K, K] (row = m-layout component,
 *                               column = e3nn component); its inverse is the
 *                               transpose.  bwd: g_vec [E, 3] from g_wigner.
 *   tace_edge_rotate_in_fwd/_bwd
 *                               gather of [x_src | x_dst], the wigner bmm and
 *                               the radial weighting (oam_2026_07_05.py:769-780):
 *                               x [n_rows, K, C] node features (l layout),
 *                               rows_src / rows_dst (int64) the feature rows of
 *                               each edge's ends; m = W [x_src | x_dst] is
 *                               written as the block arrays m_src (first C
 *                               channels) and m_dst (last C) and, given
 *                               radial_w [E, ncomp, 2C] (ncomp = (lmax+1)
 *                               (lmax+2)/2 components, shared by the +m and -m
 *                               rows), m_w = radial_w[comp(r)] m with 2C
 *                               channels.
 *                               Rows outside [0, n_rows) read as zeros.  bwd
 *                               (absent output gradients = zero): per-edge
 *                               g_x_src, g_x_dst [E, K, C] (the caller sums
 *                               them into the rows), g_wigner [E, K, K] and,
 *                               if g_radial_w is given, g_radial_w.
 *   tace_tece_score_fwd/_bwd    OAM20260705Convolution._complex_qk_attention
 *                               (_e3nn/archive/oam_2026_07_05.py:699-754): q, k
 *                               block arrays with C channels, radial_proj [E, 2H]
 *                               (bias | phase logits), tscale[H] = attention
 *                               scale x temperature -> score [E, H]; the
 *                               per-head width C/H divides 64 or is a
 *                               multiple of 64.
 *   tace_tece_edge_ace_fwd/_bwd gate + complex edge-ACE product
 *                               (oam_2026_07_05.py:782-790; SO2Gate, and
 *                               uuuSO2TensorProduct 312-516): out = u + g u +
 *                               ece(u, v, c) on the stacked SO(2) GEMM
 *                               outputs, n = lmax+1, A = hidden, P = number of
 *                               edge-ACE paths: y0 [E, P n A (coef logits) |
 *                               n A (v, m=0) | n (lmax+1) A (gate logits) |
 *                               n A (u, m=0)], y_m [2E, n A (v) | n A (u)] for
 *                               m = 1..lmax (row 2e = +m, 2e+1 = -m); out o0
 *                               [E, n A], o_m [2E, n A].  Pointers past lmax
 *                               are ignored.  bwd: g_y* from g_o*.
 *   tace_graph_softmax_fwd/_bwd GraphSoftmax (softmax.py:80-114) over each
 *                               receiver's in-edges (receiver CSR rowptr/eid),
 *                               no rescale: alpha [E, H].
 *   tace_tece_rotate_out_fwd/_bwd
 *                               alpha-weighted wigner_inv product and
 *                               scatter_sum to receivers
 *                               (oam_2026_07_05.py:799-823): m (block array,
 *                               C channels) ->
 *                               out in the group-major layout of C x (0..lmax)
 *                               at rows node_map[n]; bwd (per edge, dst[e] =
 *                               receiver node id, int64) gives g_m, g_alpha
 *                               and g_wigner. */
int tace_edge_wigner_fwd(int dtype, const void* vec, int64_t n_edges, int32_t lmax, void* wigner, void* stream);
int tace_edge_wigner_bwd(int dtype, const void* vec, const void* g_wigner, int64_t n_edges, int32_t lmax,
                         void* g_vec, void* stream);
int tace_edge_rotate_in_fwd(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                            const int64_t* rows_dst, const void* radial_w, int64_t n_rows, int64_t n_edges,
                            int32_t lmax, int32_t channels, const void* const* m_src, const void* const* m_dst,
                            const void* const* m_w, void* stream);
int tace_edge_rotate_in_bwd(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                            const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                            const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows, int64_t n_edges,
                            int32_t lmax, int32_t channels, void* g_x_src, void* g_x_dst, void* g_wigner,
                            void* g_radial_w, int32_t accumulate_wigner, void* stream);
/* accumulate_wigner != 0: g_wigner[e] += this gradient on the Wigner
 * matrix's l blocks, the entries off the blocks left as they are (the
 * caller's zeros, as tace_tece_rotate_out_bwd writes them), so the two
 * rotations' Wigner gradients sum without another pass; 0: g_wigner is
 * written, zeros off the blocks.
 * tace_edge_rotate_in_bwd_runs: tace_edge_rotate_in_bwd for edges in
 * receiver-CSR order, 4 (lmax+1)^2 channels values of at most 64 KB: the
 * receiver rows of the four edges a workgroup holds (positions 4 b .. 4 b + 3)
 * are summed per run of equal rows_dst in edge order and written once, at the
 * run's first position of g_x_dst_runs [E, K, C]; the other positions are not
 * written.  tace_rows_accumulate_runs (run = 4) then sums them per receiver:
 * the receiver half of the index_add of oam_2026_07_05.py:769-771's gather,
 * run backwards, with a quarter of the per-edge rows. */
int tace_edge_rotate_in_bwd_runs(int dtype, const void* x, const void* wigner, const int64_t* rows_src,
                                 const int64_t* rows_dst, const void* radial_w, const void* const* g_m_src,
                                 const void* const* g_m_dst, const void* const* g_m_w, int64_t n_rows,
                                 int64_t n_edges, int32_t lmax, int32_t channels, void* g_x_src, void* g_x_dst_runs,
                                 void* g_wigner, void* g_radial_w, int32_t accumulate_wigner, void* stream);
int tace_tece_score_fwd(int dtype, const void* const* q, const void* const* k, const void* radial_proj,
                        const void* tscale, int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads,
                        void* score, void* stream);
int tace_tece_score_bwd(int dtype, const void* const* q, const void* const* k, const void* radial_proj,
                        const void* tscale, const void* g_score, int64_t n_edges, int32_t lmax, int32_t channels,
                        int32_t heads, const void* const* g_q, const void* const* g_k, void* g_radial_proj,
                        void* stream);
int tace_tece_edge_ace_fwd(int dtype, const void* y0, const void* y1, const void* y2, const void* y3,
                           int64_t n_edges, int32_t lmax, int32_t hidden, void* o0, void* o1, void* o2, void* o3,
                           void* stream);
int tace_tece_edge_ace_bwd(int dtype, const void* y0, const void* y1, const void* y2, const void* y3,
                           const void* g_o0, const void* g_o1, const void* g_o2, const void* g_o3, int64_t n_edges,
                           int32_t lmax, int32_t hidden, void* g_y0, void* g_y1, void* g_y2, void* g_y3,
                           void* stream);
int tace_graph_softmax_fwd(int dtype, const void* score, const int32_t* rowptr, const int32_t* eid, int64_t n_nodes,
                           int32_t heads, void* alpha, void* stream);
int tace_graph_softmax_bwd(int dtype, const void* alpha, const void* g_alpha, const int32_t* rowptr,
                           const int32_t* eid, int64_t n_nodes, int32_t heads, void* g_score, void* stream);
/* tace_tece_rotate_out_fwd writes out with out_rows rows (0: n_nodes; other
 * values need node_map, each of the n_nodes receivers going to row
 * node_map[n] < out_rows): a receiver chunk's sums go straight into the
 * whole batch's output.  tace_tece_rotate_out_bwd reads g_out with n_nodes
 * rows the same way (the whole batch's, with a chunk's edges and dst). */
int tace_tece_rotate_out_fwd(int dtype, const void* const* m, const void* alpha, const void* wigner,
                             const int32_t* rowptr, const int32_t* eid, const int32_t* node_map, int64_t n_nodes,
                             int64_t out_rows, int32_t lmax, int32_t channels, int32_t heads, void* out,
                             void* stream);
int tace_tece_rotate_out_bwd(int dtype, const void* const* m, const void* alpha, const void* wigner,
                             const void* g_out, const int64_t* dst, const int32_t* node_map, int64_t n_nodes,
                             int64_t n_edges, int32_t lmax, int32_t channels, int32_t heads, const void* const* g_m,
                             void* g_alpha, void* g_wigner, void* stream);

/* ---- neighbour list (float64 positions, host cell[9] rows = lattice
 * vectors, host pbc[3]).  Edge (src=i, dst=j, S) exists iff
 * |r_j - r_i + S.cell|^2 < cutoff^2 and (i, S) != (j, 0); S = 0 on
 * non-periodic axes.  Output is grouped by receiver j (CSR):
 *   1. tace_nl_workspace_bytes -> allocate workspace
 *   2. tace_nl_count  -> counts[n] (edges per receiver)
 *   3. tace_scan_i32(counts) -> rowptr[n+1]; E = rowptr[n]
 *   4. tace_nl_fill   -> src[E] (int32), shifts[E,3] (int32) in rowptr order. */
int64_t tace_nl_workspace_bytes(int64_t n_atoms, const double* cell, const int32_t* pbc, double cutoff);
int tace_nl_count(const double* pos, int64_t n_atoms, const double* cell, const int32_t* pbc, double cutoff,
                  void* workspace, int64_t workspace_bytes, int32_t* counts, void* stream);
int tace_nl_fill(const double* pos, int64_t n_atoms, const double* cell, const int32_t* pbc, double cutoff,
                 const void* workspace, const int32_t* rowptr, int32_t* src, int32_t* shifts, void* stream);
/* The same search for a batch of structures (a collated batch of the
 * reference's per-structure get_neighborhood calls,
 * dataset/neighbour_list.py:195-298, one per structure from
 * dataset/graph.py:53-60) in one launch per phase; structures are back to back in pos and
 * node ids are batch-global (src too).  Each structure's edges are exactly
 * what tace_nl_count/_fill give for it alone, in the same order.
 *   1. tace_nl_batch_plan(plan = NULL) -> plan bytes; again with a host
 *      buffer of that size -> the plan table (per-structure geometry, atom
 *      and bin offsets), *n_atoms, *n_bins; copy it to device memory as is
 *      (the kernels trust it);
 *   2. tace_nl_batch_workspace_bytes(n_atoms, n_bins) -> allocate workspace;
 *   3. tace_nl_batch_count -> counts[n_atoms];
 *   4. tace_scan_i32(counts) -> rowptr[n_atoms+1];
 *   5. tace_nl_batch_fill -> src[E], shifts[E,3] in rowptr order.
 * sizes [n_structs] (int64), cells [n_structs, 3, 3] (rows = lattice
 * vectors), pbcs [n_structs, 3].  mode: 0 = automatic, 1 = a thread per
 * receiver, 2 = a wavefront per receiver (small structures); the result does
 * not depend on it. */
int64_t tace_nl_batch_plan(int32_t n_structs, const int64_t* sizes, const double* cells, const int32_t* pbcs,
                           double cutoff, void* plan, int64_t plan_bytes, int64_t* n_atoms, int64_t* n_bins);
int64_t tace_nl_batch_workspace_bytes(int64_t n_atoms, int64_t n_bins);
int tace_nl_batch_count(const double* pos, int64_t n_atoms, int32_t n_structs, const void* plan, int64_t n_bins,
                        void* workspace, int64_t workspace_bytes, int32_t mode, int32_t* counts, void* stream);
int tace_nl_batch_fill(const double* pos, int64_t n_atoms, int32_t n_structs, const void* plan, int64_t n_bins,
                       const void* workspace, int64_t workspace_bytes, int32_t mode, const int32_t* rowptr,
                       int32_t* src, int32_t* shifts, void* stream);
/* Segmented row sum added into out: for each segment s < n_segments,
 * out[target[s], :] += sum over k in [rowptr[s], rowptr[s+1]) of
 * rows[slot[k], :] (slot NULL: rows[k]; target NULL: target[s] = s), rows of
 * `width` values, summed in slot order (deterministic, no atomics).  A target
 * row may appear in at most one segment of a call.  It sums the per-edge
 * grad_x rows of the TECE rotate-in backward over each receiver (receiver
 * CSR) and each sender (a sender CSR) -- the index_add of
 * oam_2026_07_05.py:769-771's gather, run backwards.  rowptr, slot and target
 * are trusted device arrays (values within [0, n_rows) and [0, n_out_rows)). */
int tace_rows_accumulate(int dtype, const void* rows, int64_t n_rows, int64_t width, const int32_t* rowptr,
                         const int32_t* slot, const int32_t* target, int64_t n_segments, void* out,
                         int64_t n_out_rows, void* stream);
/* A narrow linear map of rows: out[r, j] = bias[j] + sum_i x[r, i] m[i, j]
 * for r < n_rows, x [n_rows, k], m [k, n] row-major, bias [n] or NULL, out
 * [n_rows, n] (1 <= k, n <= 64), summed in i order.  The TECE radial
 * projection radial_proj(R) (oam_2026_07_05.py:678-682, 699-754: [E, num_radial]
 * -> [E, 2 H]) and its input gradient (m = the weight untransposed), which a
 * library GEMM runs as one launch per call at 8 x 8 sizes. */
int tace_narrow_linear(int dtype, const void* x, int64_t n_rows, int32_t k, const void* m, const void* bias,
                       int32_t n, void* out, void* stream);
/* Per-graph sums of node rows: out[g, :] = sum over k in [ptr[g], ptr[g+1])
 * of values[k, :] (rows of `width` values, 0 < width <= 4096; out is
 * overwritten), in a fixed order that depends only on the graph's size, so
 * the same bits on every run.  Replaces the atomics of scatter_sum(x, batch)
 * (tace/utils/torch_scatter.py:43-62) for the graph energies
 * (tace/models/_e3nn/tace.py:364, 416) and for the backward of the strain
 * gather sym[batch] (tace/models/utils.py:50-79).  ptr is a trusted device
 * array of n_graphs + 1 non-decreasing offsets within [0, n_rows]. */
int tace_graph_sum(int dtype, const void* values, int64_t n_rows, int64_t width, const int64_t* ptr,
                   int64_t n_graphs, void* out, void* stream);
/* tace_rows_accumulate over the CSR positions themselves (slot NULL) that
 * only reads each segment's first position and the multiples of `run`
 * inside it: the run sums tace_edge_rotate_in_bwd_runs writes (run = 4). */
int tace_rows_accumulate_runs(int dtype, const void* rows, int64_t n_rows, int64_t width, const int32_t* rowptr,
                              const int32_t* target, int64_t n_segments, int32_t run, void* out, int64_t n_out_rows,
                              void* stream);
/* The TECE SO(2) linears under bf16 channel mixing
 * (oam_2026_07_05.py:138-247, SO2_m0_Linear / SO2_m_Linear per m block, and
 * their input gradients with the transposed weights):
 *   out[i, j] = sum_k a[i, k] B[k, j] (+ bias[j])   for i < m, j < n
 * a bf16 [m, k] with row stride lda (elements, >= k), out float32 [m, n] with
 * row stride ldo (>= n), bias float32 [n] or NULL; products of bf16 values
 * summed in float32.  B [k, n] bf16 is passed in MFMA fragment order: per
 * 16-column block cb < ceil(n / 16) and 32-k step s < ceil(k / 32), the 512
 * values B[32 s + 8 g + e][16 cb + f] (f < 16, g < 4, e < 8; zeros past k and
 * n) at b_frag[(cb ceil(k / 32) + s) 512 + (16 g + f) 8 + e], 16-byte
 * aligned.  0 < k <= 2048. */
int tace_so2_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b_frag, const float* bias, float* out,
                       int64_t ldo, int64_t m, int32_t n, int32_t k, void* stream);
/* The same product for large k (0 < k <= 65536): a 128-row x 256-column
 * output tile per workgroup with A staged through LDS in 64-k steps, so B is
 * read once per 128 rows whatever k (tace_so2_gemm_bf16 holds all of a row
 * tile's k in LDS, 32-128 rows).  Same arguments and layout; float32 sums of
 * the same bf16 products in k order. */
int tace_so2_gemm_bf16_kt(const uint16_t* a, int64_t lda, const uint16_t* b_frag, const float* bias, float* out,
                          int64_t ldo, int64_t m, int32_t n, int32_t k, void* stream);
/* Edge pairs of a neighbour list in receiver-CSR form (rowptr, eid as for
 * the tensor products; src [E] senders, shifts [E, 3] int32 periodic shifts,
 * by edge id): the reverse of edge e (i -> j, S) is the edge j -> i with
 * shift -S (the full list of dataset/neighbour_list.py:195-298 holds both).
 * Each pair gets one row, numbered in order of its lower edge id; an edge
 * without a reverse gets a row of its own.  Outputs: w_rows [E] (the row of
 * every edge), row_edges [E] and row_partner [E] (for the first n_rows rows:
 * the lower edge id and its partner, -1 for none).  work: TACE_EDGE_PAIRS_WORK(E)
 * int32; n_rows is left in work[3 E]. */
#define TACE_EDGE_PAIRS_WORK(E) (3 * (E) + 2 * (((E) + 1023) / 1024) + 4)
int tace_edge_pairs(const int32_t* rowptr, const int32_t* eid, const int32_t* src, const int32_t* shifts,
                    int64_t n_nodes, int64_t n_edges, int32_t* work, int32_t* w_rows, int32_t* row_edges,
                    int32_t* row_partner, void* stream);
/* exclusive prefix sum: out[0] = 0, out[i+1] = out[i] + counts[i], i < n */
int tace_scan_i32(const int32_t* counts, int64_t n, int32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TACE_HIP_H */
