/*
 * xnn_amd.h -- C ABI of the MI355X (gfx950) per-edge hot path of xnn.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream; nothing here knows about torch. All memory (outputs and workspace)
 * is allocated by the caller. Calls are asynchronous on `stream` and return a
 * status code:
 *   XNN_OK        0  launched
 *   XNN_EINVAL    1  bad argument (message in xnn_last_error())
 *   XNN_ECAPACITY 2  an output capacity was too small (the needed count is written)
 *   XNN_EHIP      3  a HIP launch/runtime error
 *
 * Conventions shared by all entry points (they follow the reference):
 *   - edges are directed, `src` = sender, `dst` = receiver; the edge vector is
 *     r_e = pos[dst] - pos[src] + shift_e @ cell            (atomic_data.py:371-418)
 *   - `shift` is the integer image shift packed as three signed 10-bit fields
 *     (x | y << 10 | z << 20), range [-512, 511] per axis.
 *   - `pos` and `cell` share the geometry dtype; per-edge/per-node features use
 *     the compute dtype. Dtype codes: XNN_F32 = 0, XNN_F64 = 1.
 *   - CSR "plans": ptr_dst (N+1) and optional perm_dst (E) list the edges of
 *     every receiver; ptr_src/perm_src list the edges of every sender. A NULL
 *     perm means the edges are already in that order.
 *   - `batch` (N,) int32 is the structure of every atom; `cell` is (B,3,3) or
 *     NULL for molecules (then shifts are ignored).
 */
#ifndef XNN_AMD_H
#define XNN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* xnn_stream_t; /* == hipStream_t */

enum { XNN_OK = 0, XNN_EINVAL = 1, XNN_ECAPACITY = 2, XNN_EHIP = 3 };
enum { XNN_F32 = 0, XNN_F64 = 1 };
enum { XNN_BASIS_BESSEL = 0, XNN_BASIS_GAUSSIAN = 1 };
/* Envelopes multiply the radial basis and are zero for r >= cutoff (cutoff.py:41, 125);
 * XNN_ENV_NONE is the unit step (r < cutoff) with no smooth decay. */
enum { XNN_ENV_POLYNOMIAL = 0, XNN_ENV_COSINE = 1, XNN_ENV_NONE = 2 };

/* Last error message of the calling thread ("" if none). */
const char* xnn_last_error(void);
/* ABI version (bumped on any signature change). */
int xnn_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Radial basis x envelope and spherical harmonics of one edge.              */
/*   basis  : BesselRBF      common/featurizers/radial.py:187-268           */
/*            GaussianRBF    common/featurizers/radial.py:15-75             */
/*   envelope: PolynomialCutoff common/featurizers/cutoff.py:83-125         */
/*             CosineCutoff     common/featurizers/cutoff.py:10-41          */
/*   sh     : e3nn SphericalHarmonics(normalize=True, "component"), y polar  */
/*            gnn/featurizers/spherical.py:91-93, 135-138                   */
typedef struct {
  int32_t n_rbf;         /* K                                               */
  int32_t basis;         /* XNN_BASIS_*                                     */
  int32_t envelope;      /* XNN_ENV_*                                       */
  int32_t poly_p;        /* polynomial envelope degree p                    */
  int32_t l_max;         /* 0..3 (sh has (l_max+1)^2 columns)               */
  int32_t sh_sign;       /* +1: Y(r_e); -1: Y(-r_e) (NequIP, nequip.py:722) */
  double cutoff;         /* rc                                              */
  double rbf_prefactor;  /* Bessel normalization                            */
  double gaussian_gamma; /* Gaussian exponent                               */
} xnn_featurize_params;

/* Per-edge geometry and features, edge-parallel, in the edges' own order.
 * Replaces AtomicGraph.edge_vectors (atomic_data.py:371-418) followed by
 * SphericalHarmonicEdgeEmbedding.embed (gnn/featurizers/spherical.py:115-138).
 * The edge vectors come either from `vec_in` ((E,3), compute dtype: embed(vec)) or,
 * when vec_in is NULL, from pos/cell/src/dst/shift.
 * rbf_table: (K,) Bessel frequencies (BesselRBF.freqs) or Gaussian centers, compute dtype.
 * Outputs (each nullable): vec (E,3), length (E,), sh (E,(l_max+1)^2), radial (E,K). */
int xnn_edge_featurize(int geom_dtype, int compute_dtype, const void* vec_in,
                       const void* pos, int64_t n_nodes,
                       const void* cell, int64_t n_graphs, const int32_t* batch,
                       const int32_t* src, const int32_t* dst, const int32_t* shift,
                       int64_t n_edges, const xnn_featurize_params* prm, const void* rbf_table,
                       void* vec, void* length, void* sh, void* radial, xnn_stream_t stream);

/* Chain rule of xnn_edge_featurize to the edge vectors: g_e = dL/dr_e (E,3),
 * compute dtype. Every upstream gradient is nullable (zero):
 *   d_vec (E,3), d_length (E,), d_sh (E,L), d_radial (E,K), g_extra (E,3) (added as is).
 * Replaces the autograd backward of spherical.py:135-138 and radial.py/cutoff.py. */
int xnn_edge_featurize_backward(int geom_dtype, int compute_dtype, const void* vec_in,
                                const void* pos, int64_t n_nodes,
                                const void* cell, int64_t n_graphs, const int32_t* batch,
                                const int32_t* src, const int32_t* dst, const int32_t* shift,
                                int64_t n_edges, const xnn_featurize_params* prm,
                                const void* rbf_table, const void* d_vec, const void* d_length,
                                const void* d_sh, const void* d_radial, const void* g_extra,
                                void* g_edge, xnn_stream_t stream);

/* Deterministic reduction of per-edge vector gradients onto atoms and cells.
 * Replaces _EdgeVectors.backward (atomic_data.py:452-467): grad_pos[i] =
 * sum_{dst=i} g_e - sum_{src=i} g_e (written, geometry dtype), and, when
 * cell_partial != NULL, cell_partial[i] = sum_{dst=i} shift_e (x) g_e as
 * (N,3,3) float64 (sum it per structure with xnn_segment_reduce_f64 to get
 * grad_cell = shifts^T g). When virial_partial != NULL, virial_partial[i] =
 * sum_{dst=i} r_e (x) g_e (N,3,3) float64 from the edge vectors vec (E,3, compute
 * dtype): summed per structure it is M = sum_e r_e (x) dE/dr_e, and sym(M) is the
 * strain derivative of ForceStressOutput (outputs.py:166-216) for an energy that
 * depends on positions and cell only through the edge vectors.
 * visit (N int32, nullable): the order in which atoms are taken, a spatial order (the
 * results do not depend on it); consecutive runs of it go to one XCD.
 * No float atomics: rows are walked in CSR order. */
int xnn_edge_force_reduce(int geom_dtype, int compute_dtype, const void* g_edge, int64_t n_edges,
                          const int32_t* ptr_dst, const int32_t* perm_dst,
                          const int32_t* ptr_src, const int32_t* perm_src,
                          const int32_t* shift, const int32_t* visit, int64_t n_nodes,
                          void* grad_pos, double* cell_partial, const void* vec,
                          double* virial_partial, xnn_stream_t stream);

/* xnn_edge_force_reduce for ONE structure with its strain derivative: grad_pos as above,
 * and virial (3,3) of virial_dtype (XNN_F32 / XNN_F64) = sym(sum_e r_e (x) g_e), the value
 * of xnn_edge_force_reduce's virial_partial followed by xnn_virial_reduce(symmetrize = 1) to
 * float64 rounding (another fixed summation order; repeated calls give the same bits). Two
 * launches: the reduction writes one 3x3 sum per block to the workspace, and a one-block
 * kernel adds them in block order. No atomics. Workspace:
 * xnn_edge_force_reduce_virial_workspace_bytes (0 for an empty structure). Replaces the same
 * _EdgeVectors.backward (atomic_data.py:452-467) plus the per-structure strain sum of
 * ForceStressOutput (outputs.py:166-216) when the batch holds one structure. */
size_t xnn_edge_force_reduce_virial_workspace_bytes(int64_t n_edges, int64_t n_nodes);
int xnn_edge_force_reduce_virial(int geom_dtype, int compute_dtype, const void* g_edge,
                                 int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                                 const int32_t* ptr_src, const int32_t* perm_src,
                                 const int32_t* visit, int64_t n_nodes, void* grad_pos,
                                 const void* vec, int virial_dtype, void* virial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* The strain deformation of ForceStressOutput (outputs.py:166-180): with
 * S_b = (strain_b + strain_b^T) / 2 (strain (B,3,3), geometry dtype),
 * pos_out[i] = pos[i] (I + S_batch[i]) and cell_out[b] = cell[b] (I + S_b) (cell nullable).
 * batch (N) int32 may be NULL for one structure. */
int xnn_strain_apply(int geom_dtype, const void* pos, int64_t n_nodes, const int32_t* batch,
                     const void* cell, int64_t n_graphs, const void* strain, void* pos_out,
                     void* cell_out, xnn_stream_t stream);

/* Backward of xnn_strain_apply for upstream g_pos (N,3) and g_cell (B,3,3):
 * grad_pos = g_pos (I + S)^T, grad_cell = g_cell (I + S)^T, partial[i] = pos[i] (x) g_pos[i]
 * (N,3,3) float64 (sum per structure with xnn_segment_reduce_f64) and
 * cell_term[b] = cell[b]^T g_cell[b] (B,3,3) float64; the strain gradient is
 * sym(sum_i partial_i + cell_term_b). */
int xnn_strain_apply_backward(int geom_dtype, const void* pos, int64_t n_nodes,
                              const int32_t* batch, const void* cell, int64_t n_graphs,
                              const void* strain, const void* g_pos, const void* g_cell,
                              void* grad_pos, void* grad_cell, double* partial,
                              double* cell_term, xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Fused SH message aggregation: out[i,c,lm] = sum_{e: dst=i} phi[e,c] * Y_lm(sign r_e)
 * over the receiver CSR. Y is recomputed from positions in registers (never stored).
 * This is the uvu tensor product of scalar edge weights with Y followed by
 * scatter_sum to receivers: gnn/fast/conv.py:137-143 + common/models/ops.py:403-448.
 * phi (E,C) f32, out (N,C,L) f32 with L=(l_max+1)^2, C <= 256. The edge vectors
 * come from vec_in ((E,3) f32) or, when it is NULL, from pos/cell/src/shift. */
int xnn_sh_message_sum(int geom_dtype, const float* vec_in, const void* pos, int64_t n_nodes,
                       const void* cell, int64_t n_graphs, const int32_t* batch,
                       const int32_t* src, const int32_t* shift, int64_t n_edges,
                       const int32_t* ptr_dst, const int32_t* perm_dst,
                       int32_t l_max, int32_t sh_sign, int32_t n_channels,
                       const float* phi, float* out, xnn_stream_t stream);

/* Backward of xnn_sh_message_sum: d_phi[e,c] = sum_lm d_out[dst,c,lm] Y_lm(e)
 * and g_vec[e] = dL/dr_e through Y (nullable). d_phi (E,C) f32, g_vec (E,3) f32. */
int xnn_sh_message_sum_backward(int geom_dtype, const float* vec_in, const void* pos,
                                int64_t n_nodes,
                                const void* cell, int64_t n_graphs, const int32_t* batch,
                                const int32_t* src, const int32_t* shift, int64_t n_edges,
                                const int32_t* ptr_dst, const int32_t* perm_dst,
                                int32_t l_max, int32_t sh_sign, int32_t n_channels,
                                const float* phi, const float* d_out, float* d_phi,
                                float* g_vec, xnn_stream_t stream);

/* The same aggregation with the edge weights formed by a linear layer in the kernel:
 * phi[e,c] = sum_k h[e,k] W[k,c], the last layer of the edge-weight network
 * (gnn/fast/conv.py:137-143 takes the weights from the radial network; the product
 * and the receiver sum as in xnn_sh_message_sum). The kernel takes the same sum in the
 * other order, A_i = W^T sum_{dst(e)=i} h_e (x) Y_e (the K x L feature rows summed per
 * receiver, then the linear layer per atom), so phi is never formed. h (E,K) f32 with
 * K = n_features in [1, 8],
 * W (K,C) f32 with C = n_channels in {32, 64, 128}, l_max in [1, 3]; out (N,C,L) f32,
 * 16-byte aligned. Other shapes return XNN_EINVAL (use xnn_sh_message_sum). */
int xnn_sh_linear_message_sum(int geom_dtype, const float* vec_in, const void* pos,
                              int64_t n_nodes, const void* cell, int64_t n_graphs,
                              const int32_t* batch, const int32_t* src, const int32_t* shift,
                              int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                              int32_t l_max, int32_t sh_sign, int32_t n_features,
                              int32_t n_channels, const float* h, const float* W, float* out,
                              xnn_stream_t stream);

/* Backward of xnn_sh_linear_message_sum with respect to h and the edge vectors:
 * d_h[e,k] = sum_c (sum_lm d_out[dst,c,lm] Y_lm(e)) W[k,c] (written) and g_vec (E,3)
 * (nullable; h may be NULL when g_vec is). d_W is not formed here: it is
 * h^T d_phi with d_phi from xnn_sh_message_sum_backward. d_out 16-byte aligned. */
int xnn_sh_linear_message_sum_backward(int geom_dtype, const float* vec_in, const void* pos,
                                       int64_t n_nodes, const void* cell, int64_t n_graphs,
                                       const int32_t* batch, const int32_t* src,
                                       const int32_t* shift, int64_t n_edges,
                                       const int32_t* ptr_dst, const int32_t* perm_dst,
                                       int32_t l_max, int32_t sh_sign, int32_t n_features,
                                       int32_t n_channels, const float* h, const float* W,
                                       const float* d_out, float* d_h, float* g_vec,
                                       xnn_stream_t stream);

/* Featurizer, edge-weight linear layer and aggregation in one kernel: h is the
 * enveloped radial basis of the edge length, h[e,k] = rbf_k(|r_e|) envelope(|r_e|)
 * (SphericalHarmonicEdgeEmbedding.forward, gnn/featurizers/spherical.py:135-138, whose
 * radial part feeds the edge-weight network), evaluated per lane in the kernel;
 * A[i,c,lm] = sum_{dst(e)=i} (h_e W)[c] Y_lm(sh_sign r_e) as in xnn_sh_linear_message_sum.
 * prm gives the basis, envelope, cutoff, l_max in [1, 3] and sh_sign; n_rbf = K in
 * [1, 8]; rbf_table (K) f32 (Bessel frequencies or Gaussian centers). Neither h nor
 * phi is stored. out (N,C,L) f32, 16-byte aligned. */
int xnn_sh_radial_message_sum(int geom_dtype, const float* vec_in, const void* pos,
                              int64_t n_nodes, const void* cell, int64_t n_graphs,
                              const int32_t* batch, const int32_t* src, const int32_t* shift,
                              int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                              const xnn_featurize_params* prm, const float* rbf_table,
                              int32_t n_channels, const float* W, float* out,
                              xnn_stream_t stream);

/* xnn_sh_radial_message_sum followed by the linear per-atom readout of the node rows,
 * in the same kernel: node_energy[i] = sum_{c,lm} U[c,lm] A[i,c,lm] + bias[z[i]] (bias
 * NULL: no bias; an index z outside [0, n_bias) gives NaN), so the (N,C,L) rows never
 * reach memory. It fuses the aggregation (gnn/fast/conv.py:137-143, ops.py:403-448) with
 * a model's linear energy readout before aggregate_energy (common/models/base.py:161-180);
 * the reference has no single counterpart. The kernels take E_i = sum_{dst(e)=i}
 * h_e^T (W U) Y_e + bias[z_i], the same sum with W U (K x L) formed once per block.
 * U (C,L) f32, z (N) int64, bias (n_bias) f32, node_energy (N) f32. Parameter gradients
 * are not formed. */
int xnn_sh_radial_message_energy(int geom_dtype, const float* vec_in, const void* pos,
                                 int64_t n_nodes, const void* cell, int64_t n_graphs,
                                 const int32_t* batch, const int32_t* src, const int32_t* shift,
                                 int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                                 const xnn_featurize_params* prm, const float* rbf_table,
                                 int32_t n_channels, const float* W, const float* U,
                                 const int64_t* z, const float* bias, int64_t n_bias,
                                 float* node_energy, xnn_stream_t stream);

/* Backward of xnn_sh_radial_message_energy with respect to the edge vectors for the
 * per-atom cotangent g (N) f32 of node_energy (g_stride 1, or 0: one value for every
 * atom): per edge g_i ((W U) Y_e, (W U)^T h_e) in (d h_e, dY_e), chained to the edge
 * vector. g_vec (E,3) f32 (written). */
int xnn_sh_radial_message_energy_backward(int geom_dtype, const float* vec_in, const void* pos,
                                          int64_t n_nodes, const void* cell, int64_t n_graphs,
                                          const int32_t* batch, const int32_t* src,
                                          const int32_t* shift, int64_t n_edges,
                                          const int32_t* ptr_dst, const int32_t* perm_dst,
                                          const xnn_featurize_params* prm,
                                          const float* rbf_table, int32_t n_channels,
                                          const float* W, const float* U, const float* g,
                                          int64_t g_stride, float* g_vec, xnn_stream_t stream);

/* xnn_sh_radial_message_energy_backward that also writes each edge's share of its receiver's
 * readout, edge_energy[e] = (phi_e U) . Y_e = h_e^T (W U) Y_e (E) f32, so that node_energy[i] = bias[z[i]] + sum_{dst(e)=i} edge_energy[e]
 * without the forward launch: energies and forces from one pass, as the reference's fused
 * energy-and-force evaluations return them (gnn/fast/conv.py:137-143 with the readout of
 * common/models/base.py:161-180). g_vec is the gradient for the cotangent g as in the
 * backward; a receiver's edges scale with its own cotangent. */
int xnn_sh_radial_message_energy_forces(int geom_dtype, const float* vec_in, const void* pos,
                                        int64_t n_nodes, const void* cell, int64_t n_graphs,
                                        const int32_t* batch, const int32_t* src,
                                        const int32_t* shift, int64_t n_edges,
                                        const int32_t* ptr_dst, const int32_t* perm_dst,
                                        const xnn_featurize_params* prm,
                                        const float* rbf_table, int32_t n_channels,
                                        const float* W, const float* U, const float* g,
                                        int64_t g_stride, float* g_vec, float* edge_energy,
                                        xnn_stream_t stream);

/* Node energies from the edges' shares of xnn_sh_radial_message_energy_forces:
 * node_energy[i] = bias[z[i]] + sum over the CSR row i (ptr_dst, perm_dst as for the message
 * kernels) of edge_energy, f32; bias NULL: none; an index z outside [0, n_bias) gives NaN.
 * The readout's aggregation of a fused energy-and-force pass (common/models/base.py:161-180);
 * the reference forms it from the forward's rows instead. */
int xnn_node_energy_from_edges(const float* edge_energy, const int32_t* ptr_dst,
                               const int32_t* perm_dst, int64_t n_nodes, const int64_t* z,
                               const float* bias, int64_t n_bias, float* node_energy,
                               xnn_stream_t stream);

/* Backward of xnn_sh_radial_message_sum with respect to the edge vectors, through the
 * harmonics and the radial basis: g_vec (E,3) f32 = dL/dr_e (written, not added).
 * Parameter gradients (W, rbf_table) are not formed: the caller uses
 * xnn_edge_featurize + xnn_sh_linear_message_sum(_backward) when it trains them. */
int xnn_sh_radial_message_sum_backward(int geom_dtype, const float* vec_in, const void* pos,
                                       int64_t n_nodes, const void* cell, int64_t n_graphs,
                                       const int32_t* batch, const int32_t* src,
                                       const int32_t* shift, int64_t n_edges,
                                       const int32_t* ptr_dst, const int32_t* perm_dst,
                                       const xnn_featurize_params* prm, const float* rbf_table,
                                       int32_t n_channels, const float* W, const float* d_out,
                                       float* g_vec, xnn_stream_t stream);

/* Hidden layers of a per-edge radial network in one pass over the edges:
 * s_0 = x (n_rows, n_in), s_n = silu(scales[n-1] * s_{n-1} @ W_n), out = s_{n_layers}
 * (n_rows, widths[n_layers-1]), float32 throughout (products without reduced-precision
 * inputs). W_n row-major (widths[n-2] or n_in, widths[n-1]); weights, widths and scales are
 * host arrays of n_layers entries (weights holds device pointers). 1 <= n_layers <= 3,
 * n_in <= 32, widths <= 128; x, out 16-byte aligned. Replaces FusedHidden.forward
 * (gnn/fast/radial_kernels.py:43-58, 110-119; RadialNet._hidden_fused, gnn/models/
 * blocks.py:289-292, with the layer factors of RadialNet._plan, blocks.py:336-365, passed
 * as scales instead of multiplied into the matrices). */
int xnn_radial_hidden(const float* x, int64_t n_rows, int n_in, int n_layers,
                      const int32_t* widths, const float* const* weights, const float* scales,
                      float* out, xnn_stream_t stream);

/* Input gradient of xnn_radial_hidden, the activations recomputed: grad_x (n_rows, n_in)
 * from grad_out (n_rows, widths[n_layers-1]). Replaces FusedHidden.backward's kernel
 * (gnn/fast/radial_kernels.py:61-80, 121-133); the weights' gradients are the caller's
 * (PyTorch products, as there). */
int xnn_radial_hidden_backward(const float* x, const float* grad_out, int64_t n_rows, int n_in,
                               int n_layers, const int32_t* widths, const float* const* weights,
                               const float* scales, float* grad_x, xnn_stream_t stream);

/* One uvu path of an equivariant convolution: node block of degree l1 (mul channels,
 * offset off1 in the node rows), edge-attribute block of degree l2 (one copy, offset off2),
 * output block of degree l3 (mul channels, offset off_out), weights off_w .. off_w + mul
 * of the weight rows, scale coef (the path normalization over the message divisor);
 * block: index of the node block the path reads (paths with one index share l1, mul and
 * off1; the backward accumulates each block's gradient over its paths). */
typedef struct {
  int32_t l1, l2, l3;
  int32_t mul;
  int32_t off1, off2, off_out, off_w;
  int32_t block;
  float coef;
} xnn_uvu_path;

/* The message step of an equivariant convolution (uvu tensor product of the gathered
 * sender features with the edge attributes under per-edge weights, summed onto the
 * receivers): out[i, p, u, k] = coef_p sum_{e: dst(e)=i} w[row(e), off_w_p + u]
 * sum_{a,b} C[a,b,k] h[src(e), off1_p + u (2 l1 + 1) + a] Y[e, off2_p + b], C the real
 * Wigner 3j tensor of (l1, l2, l3) (e3nn convention), row(e) = weight_index[e] (nullable:
 * e; rows outside [0, n_weight_rows) contribute nothing). Degrees <= 3, at most 48 paths
 * with distinct output blocks, at most 16 node blocks, dim2 <= 16, one edge-attribute
 * block per degree; receiver CSR (ptr_dst, perm_dst) of xnn_edge_plan. Output blocks of no
 * path are not written. Float32, deterministic.
 * Replaces ConvTensorProduct.conv (gnn/fast/conv.py:93-143: gather_rows + e3nn
 * TensorProduct + scatter_sum + the message divisor) for its fast-eligible products
 * (conv.py:35-45). */
int xnn_uvu_conv(const float* node_feats, int64_t n_nodes, int32_t dim1, const float* edge_attrs,
                 int32_t dim2, const float* weights, int64_t n_weight_rows, int32_t dim_w,
                 const int32_t* weight_index, const int32_t* src, int64_t n_edges,
                 const int32_t* ptr_dst, const int32_t* perm_dst, const xnn_uvu_path* paths,
                 int32_t n_paths, float* out, int32_t dim_out, xnn_stream_t stream);

/* Workspace of xnn_uvu_conv_backward when it forms grad_edge_attrs or grad_node_feats:
 * one float per edge, node block and edge-attribute column (the blocks' shares of d Y),
 * then one float per edge and node-row column up to the last column a path reads (each
 * edge's share of d h at its sender). */
size_t xnn_uvu_conv_workspace_bytes(int64_t n_edges, int32_t dim2, const xnn_uvu_path* paths,
                                    int32_t n_paths);

/* Gradients of xnn_uvu_conv from grad_out (N, dim_out), each output nullable. One walk
 * over the receiver CSR gives grad_edge_attrs (E, dim2), grad_weights (E, dim_w) per edge
 * (the caller sums the rows of shared weights) and each edge's share of d h; grad_node_feats
 * (N, dim1) is then the sum of those shares over the sender CSR (ptr_src, perm_src), in row
 * order (columns past the last one a path reads are not written; gaps between the path-read
 * blocks get zeros). */
int xnn_uvu_conv_backward(const float* node_feats, int64_t n_nodes, int32_t dim1,
                          const float* edge_attrs, int32_t dim2, const float* weights,
                          int64_t n_weight_rows, int32_t dim_w, const int32_t* weight_index,
                          const int32_t* src, const int32_t* dst, int64_t n_edges,
                          const int32_t* ptr_dst, const int32_t* perm_dst,
                          const int32_t* ptr_src, const int32_t* perm_src,
                          const xnn_uvu_path* paths, int32_t n_paths, const float* grad_out,
                          int32_t dim_out, float* grad_node_feats, float* grad_edge_attrs,
                          float* grad_weights, void* workspace, size_t workspace_bytes,
                          xnn_stream_t stream);

/* The parameters of the measured edge potential (ShEdgePotential): the featurizer
 * (host struct; its l_max, sh_sign, basis, envelope and cutoff), the radial table (K)
 * device float32, the linear layer W (K, C), the readout U (C, (l_max+1)^2) and the
 * per-element reference energies atom_ref (n_atom_ref), all device float32. */
typedef struct {
  const xnn_featurize_params* prm;
  const float* rbf_table;
  int32_t n_channels;
  const float* W;
  const float* U;
  const float* atom_ref;
  int64_t n_atom_ref;
} xnn_sh_pair_model;

/* Workspace of xnn_sh_pair_energy_forces for a step of n_nodes atoms and n_edges edges. */
size_t xnn_sh_pair_workspace_bytes(int64_t n_nodes, int64_t n_edges);

/* One MD step of the edge potential from a pair style's tensors: positions pos (N,3)
 * (geometry dtype), atomic_numbers (N) int64, the neighbor list edge_index (2,E) int64
 * (row 0 sender, row 1 receiver) with integer image shifts cell_shifts (E,3) int64
 * (nullable: none), cell (3,3) geometry dtype (NULL: a molecule), all device memory.
 * Writes the total energy to *energy_host (float64, host), node_energy (N) float32, forces
 * (N,3) geometry dtype and, when virial is not NULL, the virial W = -sym(sum_e r_e (x)
 * dE/dr_e) (3,3) float64 (the pair-style sign; W = -V sigma for the stress sigma of
 * ForceStressOutput). Synchronous: the call ends by reading the energy and the edge
 * plan's check back (invalid atom indices: XNN_EINVAL; shifts outside [-512, 511]:
 * XNN_ECAPACITY). Replaces LAMMPSWrapper.forward (common/deploy/lammps.py:83-145) and
 * TorchScriptPotential.forward_lammps (common/deploy/torchscript.py:883-921) for this
 * model, without libtorch. */
int xnn_sh_pair_energy_forces(const xnn_sh_pair_model* model, int geom_dtype, const void* pos,
                              int64_t n_nodes, const int64_t* atomic_numbers,
                              const int64_t* edge_index, const int64_t* cell_shifts,
                              int64_t n_edges, const void* cell, double* energy_host,
                              float* node_energy, void* forces, double* virial, void* workspace,
                              size_t workspace_bytes, xnn_stream_t stream);

/* Finish of a per-structure virial: out[b] = sym(M[b] + term[b]) with sym(X) = (X + X^T)/2
 * (symmetrize != 0) or M[b] + term[b], cast to dtype. M (B,3,3) float64 (from
 * xnn_segment_reduce_f64 over the per-atom partials of xnn_edge_force_reduce or
 * xnn_strain_apply_backward), term (B,3,3) float64 nullable. The strain gradient of
 * ForceStressOutput (outputs.py:166-216) is this with symmetrize = 1. */
int xnn_virial_finish(int dtype, const double* M, const double* term, int64_t n_graphs,
                      int32_t symmetrize, void* out, xnn_stream_t stream);

/* Per-structure virial from per-atom partials in one call: out[b] = sym(sum_{i in seg b}
 * partial[i] + term[b]) (symmetrize != 0) or without sym, cast to dtype (B,3,3).
 * partial (n_rows,3,3) float64 (xnn_edge_force_reduce's cell_partial / virial_partial, or
 * xnn_strain_apply_backward's partial), seg_ptr (B+1) int64, term (B,3,3) float64 nullable.
 * The same sums as xnn_segment_reduce_f64 followed by xnn_virial_finish (deterministic),
 * in two launches. Workspace: xnn_virial_reduce_workspace_bytes (never 0). */
size_t xnn_virial_reduce_workspace_bytes(int64_t n_rows, int64_t n_graphs);
int xnn_virial_reduce(int dtype, const double* partial, int64_t n_rows, const int64_t* seg_ptr,
                      int64_t n_graphs, const double* term, int32_t symmetrize, void* out,
                      void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* The stress of ForceStressOutput from the strain gradient (outputs.py:227-239):
 * stress[b] = scale * strain_grad[b] / |det cell_b| for periodic structures
 * (|det| > 1e-8 and, when pbc (B,3) bool/uint8 is given, some periodic direction),
 * zero for the molecules of a batch. strain_grad and stress (B,3,3) of dtype;
 * cell (B,3,3) of cell_dtype (f32/f64); scale = -1 takes the gradient of -E. */
int xnn_stress_finish(int dtype, const void* strain_grad, int cell_dtype, const void* cell,
                      const uint8_t* pbc, int64_t n_graphs, double scale, void* stress,
                      xnn_stream_t stream);

/* One structure's energy total and stress in one launch, for a step whose energy is the sum
 * of its node energies: energy[0] = sum_i node_energy[i] in float64 (node_dtype f32/f64; the
 * order of xnn_segment_reduce_f64's one-block sum, equal to it bit for bit for 2,048 to
 * 16,384 atoms) and stress (3,3) as xnn_stress_finish with n_graphs = 1. n_nodes at most
 * xnn_energy_stress_max_nodes(). Replaces the structure sum of the energy (base.py:161-180)
 * and the stress of ForceStressOutput (outputs.py:227-239) for one structure. */
int64_t xnn_energy_stress_max_nodes(void);
int xnn_energy_stress_finish(int node_dtype, const void* node_energy, int64_t n_nodes, int dtype,
                             const void* strain_grad, int cell_dtype, const void* cell,
                             const uint8_t* pbc, double scale, double* energy, void* stress,
                             xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Segmented sum over a CSR: out[i,:] = sum_{k in [ptr[i],ptr[i+1])} src[perm[k],:].
 * Replaces scatter_sum (common/models/ops.py:403-448) without atomics; its
 * adjoint gather_rows (ops.py:494-528) is xnn_gather_rows. dtype f32/f64. */
int xnn_segment_sum(int dtype, const void* src, int64_t n_rows, int64_t n_features,
                    const int32_t* ptr, const int32_t* perm, int64_t n_segments,
                    void* out, xnn_stream_t stream);

/* out[e,:] = src[index[e],:] (index int32). Replaces gather_rows (ops.py:494-528). */
int xnn_gather_rows(int dtype, const void* src, int64_t n_src_rows, int64_t n_features,
                    const int32_t* index, int64_t n_rows, void* out, xnn_stream_t stream);

/* Per-structure totals accumulated in float64 over contiguous node ranges
 * seg_ptr (B+1): out[b,f] = sum_{i in seg b} src[i,f]. Replaces structure_sum
 * (ops.py:531-557, fp64 accumulation) and structure_sums (ops.py:560-569).
 * A single structure is reduced in two levels over many workgroups (partials in
 * `workspace`, xnn_segment_reduce_workspace_bytes of it; NULL is allowed when that
 * size is 0); several structures take one workgroup each. Fixed summation order. */
size_t xnn_segment_reduce_workspace_bytes(int64_t n_rows, int64_t n_features,
                                          int64_t n_segments);
int xnn_segment_reduce_f64(int dtype, const void* src, int64_t n_rows, int64_t n_features,
                           const int64_t* seg_ptr, int64_t n_segments, double* out,
                           void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* xnn_segment_reduce_f64 without a workspace argument and without any allocation: the
 * partial sums live in a file-scope device array of xnn_segment_reduce_noalloc_max_bytes()
 * bytes (1 MiB; one copy per GPU, held until the process ends; its address is looked up
 * once per device on the first call). No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops).
 * Sizes whose partials exceed the array return XNN_EINVAL. Same kernels and results as
 * xnn_segment_reduce_f64. Every call on a GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams, other host threads) race. */
size_t xnn_segment_reduce_noalloc_max_bytes(void);
int xnn_segment_reduce_f64_noalloc(int dtype, const void* src, int64_t n_rows,
                                   int64_t n_features, const int64_t* seg_ptr,
                                   int64_t n_segments, double* out, xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* D4 dispersion pair terms over lattice images, float64 (no edge list: every
 * atom i meets every atom j of its structure and every translation
 * n = (n0, n1, n2) with |n_a| <= images[b, a]; vectors pos_i - pos_j + n @ cell in
 * Angstrom, lengths in bohr). Atoms of a structure are contiguous: node_ptr (B+1)
 * int64 on the device, batch (N) int32, max_atoms = the largest structure (a larger
 * one gives NaN for its atoms). species (N) int32 indexes the per-species tables.
 * cell (B,3,3) Angstrom rows or NULL (molecules). Gradients are exact derivatives of
 * the returned sums; the cell gradient comes as per-atom partials (N,3,3) whose sum
 * per structure (xnn_segment_reduce_f64) is sum n (x) dE/dr. All memory is the
 * caller's; workspace: xnn_d4_workspace_bytes(n_nodes, n_graphs, max_atoms) bytes,
 * about 800 max_atoms n_nodes for the two-body backward (per-atom partials and the
 * pair sums of every pair of tiles). The kernels walk 64-atom tiles of a spatial
 * order of each structure, every pair of two tiles once; plan is that order
 * (xnn_d4_plan on the same pos, cell and images) or NULL to build it in the call.
 * Deterministic (per-atom partials summed in a fixed order, no atomics). */
typedef struct {
  double cutoff_cn;      /* D4 CN cutoff, bohr (r <= cutoff counts)           */
  double cutoff_eeq_cn;  /* EEQ CN cutoff, bohr                               */
  double kcn, k4, k5, k6;
} xnn_d4_cn_params;

typedef struct {
  double s6, s8, a1, a2; /* BJ damping parameters                             */
  double cutoff;         /* pair cutoff, bohr (r <= cutoff counts)            */
  double width;          /* quintic switching width, bohr (<= 0: sharp)       */
} xnn_d4_pair_params;

size_t xnn_d4_workspace_bytes(int64_t n_nodes, int64_t n_graphs, int64_t max_atoms);

/* The tile plan of the D4 pair kernels for these positions and cells, built once and
 * passed to the four entry points below (no counterpart in the reference, whose CPU
 * kernel needs no ordering): plan = xnn_d4_plan_bytes(n_nodes, n_graphs) bytes of
 * device memory, the Morton order of each structure's atoms over a bin grid of their
 * (fractional, when periodic) coordinates and the first tile of each structure. */
/* images[b][c] = ceil(cutoff / interplanar spacing of axis c) of each structure's cell
 * (B,3,3 Angstrom rows, device), the translations that cover cutoff (Angstrom); 0 where
 * pbc[b][c] == 0 (pbc (B,3) uint8 or NULL: all periodic) or the cell is zero or degenerate;
 * at most 32767. Replaces the image range of neighborlist.py:74-104 for the D4 kernels. */
int xnn_d4_image_counts(const double* cell, const uint8_t* pbc, int64_t n_graphs, double cutoff,
                        int32_t* images, xnn_stream_t stream);

size_t xnn_d4_plan_bytes(int64_t n_nodes, int64_t n_graphs);
int xnn_d4_plan(const double* pos, int64_t n_nodes, const int64_t* node_ptr, int64_t n_graphs,
                const double* cell, const int32_t* images, int32_t* plan, size_t plan_bytes,
                xnn_stream_t stream);

/* cn_d4[i] = sum_{j,n: r <= cutoff_cn} k4 exp(-(|EN_i - EN_j| + k5)^2 / k6) c(r) and
 * cn_raw[i] = sum_{r <= cutoff_eeq_cn} c(r), c(r) = (1 + erf(-kcn (r - rc) / rc)) / 2,
 * rc = rcov_i + rcov_j (bohr). Replaces DFTD4.coordination_numbers (d4.py:552-591;
 * the soft cap of the EEQ CN, d4.py:589-590, is left to the caller). */
int xnn_d4_coordination(const double* pos, int64_t n_nodes, const int32_t* species,
                        const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                        int64_t max_atoms, const double* cell, const int32_t* images,
                        const int32_t* plan,
                        const double* rcov, const double* en, const xnn_d4_cn_params* prm,
                        double* cn_d4, double* cn_raw, void* workspace, size_t workspace_bytes,
                        xnn_stream_t stream);

/* Gradients of sum_i (g_cn_d4[i] cn_d4[i] + g_cn_raw[i] cn_raw[i]) (either g may be
 * NULL): grad_pos (N,3) and cell_partial (N,3,3, nullable). */
int xnn_d4_coordination_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                                 const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                                 int64_t max_atoms, const double* cell, const int32_t* images,
                                 const int32_t* plan,
                                 const double* rcov, const double* en,
                                 const xnn_d4_cn_params* prm, const double* g_cn_d4,
                                 const double* g_cn_raw, double* grad_pos, double* cell_partial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* e2[i] = sum_{j,n: r <= cutoff} -1/2 C6_ij sw(r) (s6 / (r^6 + R0^6) + s8 rr / (r^8 + R0^8)),
 * C6_ij = (3/pi) sum_w cp_w alpha_i(w) alpha_j(w) over the 23-point Casimir-Polder grid,
 * rr = 3 r4r2_i r4r2_j, R0 = a1 sqrt(rr) + a2 (hartree, bohr). alpha (N,23).
 * Replaces DFTD4.two_body_energy / pair_damping / pair_c6 (d4.py:1044-1071) and the
 * switching_function (dispersion.py:42-67). */
int xnn_d4_two_body(const double* pos, int64_t n_nodes, const int32_t* species,
                    const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                    int64_t max_atoms, const double* cell, const int32_t* images,
                    const int32_t* plan,
                    const double* r4r2, const double* alpha, const xnn_d4_pair_params* prm,
                    double* e2, void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* Gradients of sum_i g_e2[i] e2[i]: grad_pos (N,3), cell_partial (N,3,3, nullable) and
 * grad_alpha (N,23, nullable): the outputs of the reference's native pair kernel
 * (dispersion_fast/cpu.py:834-935, D4CpuFunction.backward 1356-1376) for the
 * two-body term. */
int xnn_d4_two_body_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                             const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                             int64_t max_atoms, const double* cell, const int32_t* images,
                             const int32_t* plan,
                             const double* r4r2, const double* alpha,
                             const xnn_d4_pair_params* prm, const double* g_e2, double* grad_pos,
                             double* cell_partial, double* grad_alpha, void* workspace,
                             size_t workspace_bytes, xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Large-system EEQ operator, real-space part (float64, bohr). Replaces the neighbor-list
 * kernel of EEQSystem (common/models/eeq.py:170-397, the operator of eeq_charges_large,
 * eeq.py:664; dispersion_fast/eeq.py:69 keeps it as a sparse CSR matrix):
 * matrix (N,N) = sum over lattice images n with 0 < |d| <= cutoff of
 * [erf(gamma_ij |d|) - erf(alpha |d|)] / |d|, d = pos_j + n cell - pos_i,
 * gamma_ij = (rad_i^2 + rad_j^2)^(-1/2). pos, rad and matrix are device memory; cell is
 * HOST memory, 9 doubles (rows), or NULL (a molecule: one image, alpha must be 0; the
 * cutoff may be infinite). Written, row-major, symmetric. */
int xnn_eeq_real_matrix(const double* pos, int64_t n_nodes, const double* cell,
                        const double* rad, double alpha, double cutoff, double* matrix,
                        xnn_stream_t stream);

/* Derivatives of S = sum_ij u_i matrix_ij w_j with respect to the positions, grad_pos
 * (N,3), and the cell, as per-atom rows cell_partial (N,3,3) to be summed (nullable;
 * NULL for a molecule). cell is host memory as above, the rest device memory.
 * Deterministic. */
int xnn_eeq_real_grad(const double* pos, int64_t n_nodes, const double* cell, const double* rad,
                      double alpha, double cutoff, const double* u, const double* w,
                      double* grad_pos, double* cell_partial, xnn_stream_t stream);

/* Bytes of the workspace of xnn_eeq_real_apply for n_nodes atoms and nrhs (1 or 2)
 * right-hand sides. */
int xnn_eeq_real_apply_work_size(int64_t n_nodes, int32_t nrhs, size_t* bytes);

/* out (N, nrhs) = matrix v for v (N, nrhs) row-major, nrhs 1 or 2, without forming the
 * matrix of xnn_eeq_real_matrix (the conjugate-gradient regime above LU_MAX_ATOMS,
 * common/models/eeq.py:70, 226, 325-360; dispersion_fast/eeq.py keeps the real-space
 * kernel as a sparse CSR matrix instead). Memory O(N): the screened kernel is evaluated for
 * every pair and image at every product. tiles: NULL, or (ceil(N / 256), 4) doubles, per
 * tile of 256 consecutive atoms the center and radius of a sphere holding them (in the
 * coordinates of pos); a tile pair with no lattice image within the cutoff is skipped,
 * so atoms ordered along space (a cell list's order) make a large cell's product
 * O(N x neighbors). pos, rad, tiles, v, out and work device memory, cell host memory as
 * above. Deterministic (fixed-order partial sums). */
int xnn_eeq_real_apply(const double* pos, int64_t n_nodes, const double* cell, const double* rad,
                       double alpha, double cutoff, const double* tiles, const double* v,
                       int32_t nrhs, double* out, void* work, size_t work_bytes,
                       xnn_stream_t stream);

/* One diagonal block of the blocked Cholesky factorization of the assembled operator
 * (replaces the factorization of EEQSystem._solve_lu, common/models/eeq.py:312-323, which
 * LU-factors the augmented matrix; the operator is symmetric positive definite and the
 * constraint is eliminated on the host). matrix: device, (n, n) row-major float64; the
 * block covers rows and columns [k0, k0 + b), 1 <= b <= 128, after the host has applied
 * the trailing updates of the blocks before it. Written in place: the block's factor L
 * (lower; its upper triangle zeroed), and inv (b, b) = L^-1 (row-major, lower) for the
 * panel product L21 = A21 inv^T. A pivot that is not positive and finite stores k0 + j + 1 into the
 * device int *info when that still holds 0, and leaves the block unwritten. */
int xnn_eeq_cholesky_block(double* matrix, int64_t n, int64_t k0, int64_t b, double* inv,
                           int* info, xnn_stream_t stream);

/* (L L^T) X = B in place: X (n, nrhs) row-major float64 on entry B, nrhs 1 or 2; L the
 * factor that xnn_eeq_cholesky_block left in the matrix (row-major, lower), inv_blocks the
 * inverses of its diagonal blocks (block j of rows [128 j, 128 j + b_j) at inv_blocks +
 * 128 * 128 j, row stride b_j, as xnn_eeq_cholesky_block wrote them); work: n * nrhs
 * doubles. Blocked forward and backward substitution, one launch per block and direction;
 * sums in a fixed order. Stands in for the factorized solves of the large regime
 * (eeq.py:117-140: torch.linalg.lu_solve on the LU factors), here with the Cholesky factor
 * of the symmetric operator. */
int xnn_eeq_cholesky_solve(const double* factor, int64_t n, const double* inv_blocks, double* x,
                           int32_t nrhs, double* work, xnn_stream_t stream);

/* D4 reference tables in the kernels' layout, indexed by atomic number (rows 0 ..
 * n_elements-1), device memory: nref (n_el) int32, ngw / refcn / refq (n_el, 7) with
 * ngw int32, zeff (n_el), gi = hardness x gc (n_el), refalpha (n_el, 7, 23) the
 * charge-scaled reference polarizabilities (d4.py:444-500); ga and wf the DFTD4
 * parameters (d4.py:419). */
typedef struct {
  int32_t n_elements;
  const int32_t* nref;
  const int32_t* ngw;
  const double* refcn;
  const double* refq;
  const double* zeff;
  const double* gi;
  const double* refalpha;
  double ga, wf;
} xnn_d4_alpha_tables;

/* alpha (N,23): the dynamic polarizabilities at the coordination numbers cn (N) and
 * charges q (N) -- Gaussian reference weights normalised per atom, charge scaling zeta,
 * contracted with refalpha. atomic_numbers (N) int64; one outside the tables gives NaN.
 * Replaces DFTD4.weights / polarizabilities (d4.py:984-1042) and the alpha part of the
 * reference's native d4_alpha (dispersion_fast/cpu.py:774-829). */
int xnn_d4_polarizabilities(int64_t n_nodes, const int64_t* atomic_numbers, const double* cn,
                            const double* q, const xnn_d4_alpha_tables* tables, double* alpha,
                            xnn_stream_t stream);

/* g_cn[i] = sum_k g_alpha[i,k] d alpha[i,k] / d cn[i] and g_q[i] the same in q[i] (either
 * output may be NULL): the chain rule the reference's native kernel applies with its
 * dacn / daq (dispersion_fast/cpu.py:774-829, D4CpuFunction.backward 1356-1376). */
int xnn_d4_polarizabilities_backward(int64_t n_nodes, const int64_t* atomic_numbers,
                                     const double* cn, const double* q,
                                     const xnn_d4_alpha_tables* tables, const double* g_alpha,
                                     double* g_cn, double* g_q, xnn_stream_t stream);

/* D3 two-body dispersion on the same image walk (xnn_d4_workspace_bytes covers it).
 * cn[i] = sum_{r <= cutoff_cn} 1 / (1 + exp(-kcn (rc / r - 1))), rc = rcov_i + rcov_j
 * (bohr). Replaces DFTD3.coordination_numbers (d3.py:632-642). */
int xnn_d3_coordination(const double* pos, int64_t n_nodes, const int32_t* species,
                        const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                        int64_t max_atoms, const double* cell, const int32_t* images,
                        const double* rcov, double cutoff_cn, double kcn, double* cn,
                        void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* Gradient of sum_i g_cn[i] cn[i]: grad_pos (N,3), cell_partial (N,3,3, nullable). */
int xnn_d3_coordination_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                                 const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                                 int64_t max_atoms, const double* cell, const int32_t* images,
                                 const double* rcov, double cutoff_cn, double kcn,
                                 const double* g_cn, double* grad_pos, double* cell_partial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream);

typedef struct {
  double s6, s8, a1, a2;   /* scalings; rational-damping radius a1 sqrt(C8/C6) + a2   */
  double rs6, rs8, alp;    /* zero damping: radii scalings and exponent              */
  double bet;              /* modified zero: shift; optimized power: exponent        */
  double cutoff, width;    /* pair cutoff and switching width, bohr                  */
  int32_t damping;         /* 0 bj, 1 zero, 2 mzero, 3 op                            */
} xnn_d3_pair_params;

/* e2[i] = sum_{j,n: r <= cutoff} -1/2 C6_ij sw(r) (s6 t6(r) + s8 rr t8(r)) with
 * C6_ij = sum_ab W_i[a] W_j[b] c6ref[s_i][s_j][a][b] (weights (N,7), c6ref
 * (S,S,7,7) by species), rr = 3 r4r2_i r4r2_j, and t6, t8 of the chosen damping with
 * R0 = a1 sqrt(rr) + a2 (bj, op) or rvdw[s_i][s_j] (zero, mzero; (S,S), bohr).
 * Replaces DFTD3.pair_c6 / pair_radius / two_body_energy (d3.py:651-722). */
int xnn_d3_two_body(const double* pos, int64_t n_nodes, const int32_t* species,
                    const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                    int64_t max_atoms, const double* cell, const int32_t* images,
                    const double* r4r2, const double* rvdw, const double* c6ref,
                    int32_t n_species, const double* weights, const xnn_d3_pair_params* prm,
                    double* e2, void* workspace, size_t workspace_bytes, xnn_stream_t stream);

/* Gradients of sum_i g_e2[i] e2[i]: grad_pos (N,3), cell_partial (N,3,3, nullable),
 * grad_weights (N,7, nullable; chained to the CN by the caller). */
int xnn_d3_two_body_backward(const double* pos, int64_t n_nodes, const int32_t* species,
                             const int32_t* batch, const int64_t* node_ptr, int64_t n_graphs,
                             int64_t max_atoms, const double* cell, const int32_t* images,
                             const double* r4r2, const double* rvdw, const double* c6ref,
                             int32_t n_species, const double* weights,
                             const xnn_d3_pair_params* prm, const double* g_e2, double* grad_pos,
                             double* cell_partial, double* grad_weights, void* workspace,
                             size_t workspace_bytes, xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Cell-list radius graph. Replaces build_neighbor_list (neighborlist.py:411-506):
 * same edge set (dist < cutoff in the geometry dtype), same [src,dst] and negated,
 * unwrapped shift convention; edges come grouped by receiver (CSR order).
 *
 * Call sequence (all device-side after the plan):
 *   1. xnn_radius_graph_plan(...)        host: grid shape + workspace bytes
 *   2. xnn_radius_graph_count(...)       device: per-atom neighbor counts -> row_ptr (N+1)
 *   3. caller reads row_ptr[N] (= E) and allocates outputs
 *   4. xnn_radius_graph_fill(...)        device: src, dst, shifts (+ int64 reference format)
 * The grid is in fractional coordinates: bins of normal width >= cutoff along
 * every axis (the image range of neighborlist.py:74-104 follows from it). */
typedef struct {
  int32_t nbins[3];       /* bins per axis                                      */
  int32_t reach[3];       /* bins searched on each side                          */
  int32_t periodic[3];    /* pbc flags                                           */
  int32_t has_cell;       /* 0: molecule (Cartesian grid)                        */
  double lo[3];           /* lower bound of the grid (fractional / Cartesian)     */
  double width[3];        /* bin width in the same coordinates                    */
  double inv_cell[9];     /* row-major inverse of the cell (when has_cell)        */
  int64_t n_bins;         /* product of nbins                                     */
  size_t workspace_bytes; /* bytes of device workspace the count/fill steps need  */
} xnn_grid_plan;

/* Host-only: derive the grid for one structure. `cell` (3x3, row-major, host,
 * float64) may be NULL; pbc (3) host ints; lo/hi are the host-side min/max of
 * the atoms' fractional (or Cartesian for molecules) coordinates along
 * non-periodic axes (ignored on periodic axes). */
int xnn_radius_graph_plan(int64_t n_nodes, const double* cell, const int32_t* pbc,
                          double cutoff, const double* lo, const double* hi,
                          xnn_grid_plan* plan);

/* Device: the bounds xnn_radius_graph_plan takes, in one launch, so that one read gives the
 * host all it needs: out (15 float64, device) = lo[3], hi[3] of the atoms' Cartesian
 * coordinates (cell NULL) or fractional ones pos @ inv(cell) (float64), all six NaN when a
 * coordinate is not finite, then the cell (3x3 row-major, geometry dtype on the device) as
 * float64 (zeros without a cell). Replaces the host-side min/max of neighborlist.py:411-506's
 * grid set-up. */
int xnn_radius_graph_bounds(int geom_dtype, const void* pos, int64_t n_nodes, const void* cell,
                            double* out, xnn_stream_t stream);

int xnn_radius_graph_count(int geom_dtype, const void* pos, int64_t n_nodes, const void* cell,
                           double cutoff, int32_t self_interaction, const xnn_grid_plan* plan,
                           void* workspace, int32_t* row_ptr, xnn_stream_t stream);

/* After xnn_radius_graph_count on the same plan and workspace: status (2 int32, device) =
 * (E = row_ptr[n_nodes], 1 when a position was not finite else 0), so that one read gives
 * the host the edge count and the check neighborlist.py:180-181 makes (non-finite
 * positions raise). geom_dtype is the count step's. */
int xnn_radius_graph_status(int geom_dtype, int64_t n_nodes, const xnn_grid_plan* plan,
                            const void* workspace, const int32_t* row_ptr, int32_t* status,
                            xnn_stream_t stream);

/* Writes E = row_ptr[n_nodes] edges. src/dst int32 (E), shift packed int32 (E);
 * edge_index64 (2,E) and shifts64 (E,3) int64 in the reference format are nullable
 * (src, dst and shift may be NULL together when both int64 outputs are given).
 * *overflow (device int32, nullable) is set non-zero when a packed shift field left
 * [-512, 511] (the int64 shifts stay exact). */
int xnn_radius_graph_fill(int geom_dtype, const void* pos, int64_t n_nodes, const void* cell,
                          double cutoff, int32_t self_interaction, const xnn_grid_plan* plan,
                          void* workspace, const int32_t* row_ptr, int64_t n_edges,
                          int32_t* src, int32_t* dst, int32_t* shift,
                          int64_t* edge_index64, int64_t* shifts64, int32_t* overflow,
                          xnn_stream_t stream);

/* The fill without the host knowing the edge count (replaces the same step of
 * build_neighbor_list, neighborlist.py:462-506, for a caller that sizes its outputs from
 * an earlier list, e.g. the last step of an MD run): after xnn_radius_graph_count, the
 * count E = row_ptr[n_nodes] is read on the device and, when E <= capacity, edge_index64 is
 * written as (2, E) and shifts64 as (E, 3) at the front of buffers of 2 capacity and
 * 3 capacity entries; when E > capacity nothing is written and the fill may be run again
 * with room (xnn_radius_graph_fill with n_edges = E). status (nullable, 2 int32, device)
 * receives what xnn_radius_graph_status gives: E and the non-finite flag. No host
 * synchronization. Either fill runs once per count (it counts the count step's totals
 * down), except after a capacity fill that had no room. */
int xnn_radius_graph_fill_capacity(int geom_dtype, const void* pos, int64_t n_nodes,
                                   const void* cell, double cutoff, int32_t self_interaction,
                                   const xnn_grid_plan* plan, void* workspace,
                                   const int32_t* row_ptr, int64_t capacity,
                                   int64_t* edge_index64, int64_t* shifts64, int32_t* status,
                                   xnn_stream_t stream);

/* Radius graph of a batch of small molecules (no cell): structure b owns atoms
 * [node_ptr[b], node_ptr[b+1]); every atom tests every atom of its structure.
 * Same two-step protocol as above (count -> row_ptr, then fill). Structures of
 * more than 1024 atoms are rejected (use the cell list per structure). */
/* molecules_count writes the per-atom counts to row_ptr[1..N]; follow it with
 * xnn_scan_counts to turn them into row pointers. */
int xnn_radius_graph_molecules_count(int geom_dtype, const void* pos, int64_t n_nodes,
                                     const int64_t* node_ptr, const int32_t* batch,
                                     int64_t n_graphs, double cutoff, int32_t self_interaction,
                                     int32_t* row_ptr, xnn_stream_t stream);
int xnn_radius_graph_molecules_fill(int geom_dtype, const void* pos, int64_t n_nodes,
                                    const int64_t* node_ptr, const int32_t* batch,
                                    int64_t n_graphs, double cutoff, int32_t self_interaction,
                                    const int32_t* row_ptr, int64_t n_edges, int32_t* src,
                                    int32_t* dst, int32_t* shift, int64_t* edge_index64,
                                    int64_t* shifts64, xnn_stream_t stream);

/* The k nearest in-edges of every receiver (max_neighbors; nearest_edges,
 * neighborlist.py:509-552, used by structure_to_graph, dataset.py:112-120). Two steps:
 * xnn_nearest_edges_count writes min(deg_i, k) to kept_ptr[1..N] from the receiver CSR
 * (ptr_dst of xnn_edge_plan); xnn_scan_counts turns kept_ptr into row pointers;
 * xnn_nearest_edges_fill writes the kept edge ids to keep[kept_ptr[i] + rank], rank the
 * position of the edge in its row ordered by (dist, edge id): the reference's result
 * (edges grouped by receiver, by length within each, ties in list order).
 * dist (E) float64 or float32 (dtype), perm_dst nullable (edges grouped already). */
int xnn_nearest_edges_count(const int32_t* ptr_dst, int64_t n_nodes, int32_t k, int32_t* kept_ptr,
                            xnn_stream_t stream);
int xnn_nearest_edges_fill(int dtype, const void* dist, int64_t n_edges, const int32_t* ptr_dst,
                           const int32_t* perm_dst, int64_t n_nodes, int32_t k,
                           const int32_t* kept_ptr, int64_t* keep, xnn_stream_t stream);

/* Exclusive scan helper for the two-step protocols: row_ptr[0..n] from counts
 * already stored in row_ptr[1..n] (in place). workspace: xnn_scan_workspace_bytes(n). */
size_t xnn_scan_workspace_bytes(int64_t n);
int xnn_scan_counts(int32_t* row_ptr, int64_t n, void* workspace, xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Edge plan from an arbitrary edge list: int64 edge_index (2,E) and cell_shifts
 * (E,3) -> int32 src, dst, packed shift; receiver CSR (ptr_dst, perm_dst) and
 * sender CSR (ptr_src, perm_src), both stable (edge order within a row).
 * Mirrors the orderings of common/models/csr.py:20-51. Shift fields outside
 * [-512, 511] fail with XNN_ECAPACITY (flag written to *overflow on device). */
size_t xnn_edge_plan_workspace_bytes(int64_t n_edges, int64_t n_nodes);
int xnn_edge_plan(const int64_t* edge_index, const int64_t* cell_shifts, int64_t n_edges,
                  int64_t n_nodes, int32_t* src, int32_t* dst, int32_t* shift,
                  int32_t* ptr_dst, int32_t* perm_dst, int32_t* ptr_src, int32_t* perm_src,
                  int32_t* overflow, void* workspace, size_t workspace_bytes,
                  xnn_stream_t stream);

/* D3 reference weights (N,7): w_r = exp(-wf (cn - cnref_r)^2) normalized over the
 * species' nref references (a zero norm: weight 1 on the largest-cnref references).
 * species (N) int32; nref (S) int32, refcn (S,7) species-major; wf = 4 (d3.py:465).
 * Replaces DFTD3's weights (d3.py:644-649, dispersion.py:70-121). A species outside
 * [0, S) gives NaN. */
int xnn_d3_weights(int64_t n_nodes, const int32_t* species, const double* cn,
                   int32_t n_species, const int32_t* nref, const double* refcn, double wf,
                   double* weights, xnn_stream_t stream);

/* g_cn[i] = sum_r g_weights[i,r] d w_r / d cn[i]. */
int xnn_d3_weights_backward(int64_t n_nodes, const int32_t* species, const double* cn,
                            int32_t n_species, const int32_t* nref, const double* refcn,
                            double wf, const double* g_weights, double* g_cn,
                            xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Linear per-atom readout of node rows: out[i] = bias[z[i]] + sum_f rows[i,f] w[f]
 * (rows (N,F) row-major, w (F), out (N), all in dtype; z (N) int64 and bias (n_bias)
 * both NULL for no bias; a z outside [0, n_bias) gives NaN). The readout
 * E_i = <U, A_i> + atom_ref[Z_i] of the measured edge model; no counterpart in the
 * reference's path (its models read out through their own PyTorch layers), here for
 * callers that stream large node rows once: one wave per row, deterministic. */
int xnn_node_readout(int dtype, const void* rows, int64_t n_rows, int64_t n_features,
                     const void* weights, const int64_t* z, const void* bias, int64_t n_bias,
                     void* out, xnn_stream_t stream);

/* The adjoint in rows: d_rows[i,f] = g[i * g_stride] w[f] (g_stride 0: one value for
 * every row, 1: per row). */
int xnn_node_readout_backward(int dtype, const void* g, int64_t g_stride, int64_t n_rows,
                              int64_t n_features, const void* weights, void* d_rows,
                              xnn_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Axilrod-Teller-Muto three-body dispersion (D4 and D3) over an edge list. Edges
 * edge_index (2,E) int64 [src; dst] within the three-body cutoff, both directions of
 * every pair and image; vectors edge_vec (E,3) float64 in bohr. Pair C6 of atoms x, y is
 * <feat_a[x], feat_b[y]> over k <= 32 components (feat_a, feat_b (N,k) float64; D4:
 * alpha(i w) sqrt(3 cp_w / pi)); the damping radius of a triangle is the product of the
 * three table[species, species] factors (table (S,S) float64, S <= 32; species (N)
 * int32). Energy per triangle s9 C9 (3 cos cos cos + 1) / (r r r)^3 / (1 + 6 (R0 /
 * r r r)^alp3) times the three switches, a third to each corner (dispersion.py:124-222).
 * Replaces the triplet plan and kernels of dispersion_fast/atm.py:297-535
 * (plan_triplets 318-352, _energies 380-399, _gradients 413-443) and the reference's
 * three_body_energy / three_body_energy_chunked (dispersion.py:124-222, 529-647). */
typedef struct {
  double s9;             /* three-body scale                                     */
  double alp3;           /* damping exponent: alp / 3 (D4), (alp + 2) / 3 (D3)   */
  double cutoff;         /* three-body cutoff, bohr (r_jk <= cutoff)             */
  double width;          /* switching width, bohr (<= 0: sharp cutoff)           */
} xnn_atm_params;

/* Bytes of the plan buffer for E edges and N atoms. */
int xnn_atm_plan_size(int64_t n_edges, int64_t n_atoms, size_t* bytes);

/* Sort the edges by (center, neighbor) into the plan and lay out the work. Synchronous
 * (one small device-to-host copy): info[0] = tiles of 64 upper edges of the busiest
 * center, info[1] = 1 when some center has repeated-atom triangles (periodic self-images).
 * An atom index outside [0, N) is an error. (atm.py:318-352) */
int xnn_atm_plan(const int64_t* edge_index, int64_t n_edges, int64_t n_atoms, void* plan,
                 size_t plan_bytes, int64_t* info, xnn_stream_t stream);

/* Bytes of the workspace of xnn_atm_energy (backward = 0) or of its backward (1). */
int xnn_atm_work_size(int64_t n_edges, int64_t n_atoms, int32_t k, int32_t backward,
                      size_t* bytes);

/* Per-atom ATM energies (N) in hartree, summed with atomics as reproducible head/tail
 * sums (the same bits in any order). max_tiles, has_repeats: info[0], info[1] of the plan.
 * (atm.py:84-162) */
int xnn_atm_energy(const void* plan, int64_t n_edges, int64_t n_atoms, int64_t max_tiles,
                   int64_t has_repeats, const double* edge_vec, const double* feat_a,
                   const double* feat_b, int32_t k, const int32_t* species, const double* table,
                   int32_t n_species, const xnn_atm_params* prm, double* energy, void* work,
                   size_t work_bytes, xnn_stream_t stream);

/* Gradients of sum_i grad_energy[i] E_i: grad_vec (E,3) in the input edge order, grad_fa
 * and grad_fb (N,k). (atm.py:165-294, 402-443) */
int xnn_atm_energy_backward(const void* plan, int64_t n_edges, int64_t n_atoms,
                            int64_t max_tiles, int64_t has_repeats, const double* edge_vec,
                            const double* feat_a, const double* feat_b, int32_t k,
                            const int32_t* species, const double* table, int32_t n_species,
                            const xnn_atm_params* prm, const double* grad_energy,
                            double* grad_vec, double* grad_fa, double* grad_fb, void* work,
                            size_t work_bytes, xnn_stream_t stream);

/* Bytes of the workspace of xnn_atm_energy_backward_tangent. */
int xnn_atm_tangent_work_size(int64_t n_edges, int64_t n_atoms, int32_t k, size_t* bytes);

/* Second derivatives along a direction (edge_vec_t (E,3) in the input edge order,
 * feat_a_t, feat_b_t (N,k)): energy_t (N) = the derivative of the per-atom energies along
 * it, and grad_vec_t (E,3), grad_fa_t, grad_fb_t (N,k) = the derivatives of the gradients
 * of sum_i grad_energy[i] E_i (xnn_atm_energy_backward) along it at fixed grad_energy, a
 * Hessian-vector product. Reproducible sums. Replaces the tangent kernels of
 * dispersion_fast/atm_tangents.py (_atm_forward_t, _atm_backward_t) as _ATMGrad.backward
 * calls them (dispersion_fast/atm.py:475-509). */
int xnn_atm_energy_backward_tangent(
    const void* plan, int64_t n_edges, int64_t n_atoms, int64_t max_tiles, int64_t has_repeats,
    const double* edge_vec, const double* feat_a, const double* feat_b, int32_t k,
    const int32_t* species, const double* table, int32_t n_species, const xnn_atm_params* prm,
    const double* grad_energy, const double* edge_vec_t, const double* feat_a_t,
    const double* feat_b_t, double* energy_t, double* grad_vec_t, double* grad_fa_t,
    double* grad_fb_t, void* work, size_t work_bytes, xnn_stream_t stream);

/* Measurement, no counterpart in the reference: counts[0] = edge pairs the distinct-
 * triangle walk tests, counts[1] = distinct triangles it keeps (third side within the
 * cutoff), counts[2] = repeated-atom triangle visits, for the planned edges and their
 * vectors (bohr). Synchronous; for roofline figures (flops per triangle x triangles). */
int xnn_atm_count(const void* plan, int64_t n_edges, int64_t n_atoms, int64_t max_tiles,
                  const double* edge_vec, double cutoff, int64_t* counts, xnn_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* XNN_AMD_H */
