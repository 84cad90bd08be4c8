// Pair-style entry point: one call per MD step for the measured model family (the
// equivariant edge potential behind ShEdgePotential), from the tensors a LAMMPS pair style
// holds (positions, its neighbor list as edge_index + integer shifts, atomic numbers, the
// cell) to the total and per-atom energy, the forces and the virial. It replaces
// LAMMPSWrapper.forward (common/deploy/lammps.py:83-145) and the pair-style ABI of
// TorchScriptPotential.forward_lammps (common/deploy/torchscript.py:883-921) for this model
// without libtorch: the edge plan, the fused radial-message-readout kernel and its backward,
// the edge -> atom force reduction with the edge virial, and the float64 totals, all on the
// caller's stream, in buffers carved from one caller-provided workspace.
#include <algorithm>
#include <cstdint>

#include "common.h"

namespace xnn {

__global__ void pair_fill_kernel(int32_t* __restrict__ batch, int64_t n, float* __restrict__ one,
                                 int64_t* __restrict__ seg_ptr) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) batch[i] = 0;
  if (i == 0) {
    one[0] = 1.f;
    seg_ptr[0] = 0;
    seg_ptr[1] = n;
  }
}

// forces = -dE/dpos, and the virial W = -sym(sum_e r_e (x) dE/dr_e) in float64 (the LAMMPS
// sign: positive for a repulsive system)
template <typename G>
__global__ void pair_finish_kernel(G* __restrict__ forces, int64_t n3, double* __restrict__ virial) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n3) forces[i] = -forces[i];
  if (i < 9 && virial) virial[i] = -virial[i];
}

struct PairWs {
  size_t src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, flag, plan, batch, one, seg_ptr,
      g_vec, vec, partial, seg, vir, energy, total;
  size_t plan_bytes, seg_bytes, vir_bytes;
};

static size_t pair_align(size_t x) { return (x + 255) & ~size_t(255); }

static PairWs pair_layout(int64_t n_nodes, int64_t n_edges) {
  PairWs w{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += pair_align(std::max<size_t>(bytes, 1));
    return at;
  };
  const size_t E = (size_t)n_edges, N = (size_t)n_nodes;
  w.src = take(4 * E);
  w.dst = take(4 * E);
  w.shift = take(4 * E);
  w.ptr_dst = take(4 * (N + 1));
  w.perm_dst = take(4 * E);
  w.ptr_src = take(4 * (N + 1));
  w.perm_src = take(4 * E);
  w.flag = take(4);
  w.plan_bytes = xnn_edge_plan_workspace_bytes(n_edges, n_nodes);
  w.plan = take(w.plan_bytes);
  w.batch = take(4 * N);
  w.one = take(4);
  w.seg_ptr = take(16);
  w.g_vec = take(12 * E);
  w.vec = take(12 * E);
  w.partial = take(72 * N);
  w.seg_bytes = xnn_segment_reduce_workspace_bytes(n_nodes, 1, 1);
  w.seg = take(w.seg_bytes);
  w.vir_bytes = xnn_virial_reduce_workspace_bytes(n_nodes, 1);
  w.vir = take(w.vir_bytes);
  w.energy = take(8);
  w.total = o;
  return w;
}

template <typename T>
static T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

}  // namespace xnn

using namespace xnn;

extern "C" {

size_t xnn_sh_pair_workspace_bytes(int64_t n_nodes, int64_t n_edges) {
  if (n_nodes < 0 || n_edges < 0) return 0;
  return pair_layout(n_nodes, n_edges).total;
}

int xnn_sh_pair_energy_forces(const xnn_sh_pair_model* model, int geom_dtype, const void* pos,
                              int64_t n_nodes, const int64_t* atomic_numbers,
                              const int64_t* edge_index, const int64_t* cell_shifts,
                              int64_t n_edges, const void* cell, double* energy_host,
                              float* node_energy, void* forces, double* virial, void* workspace,
                              size_t workspace_bytes, xnn_stream_t stream) {
  XNN_REQUIRE(model && model->prm && model->rbf_table && model->W && model->U && model->atom_ref,
              "NULL model field");
  XNN_REQUIRE(geom_dtype == XNN_F32 || geom_dtype == XNN_F64, "geom_dtype must be XNN_F32 or XNN_F64");
  XNN_REQUIRE(n_nodes >= 0 && n_edges >= 0, "negative size");
  XNN_REQUIRE(energy_host, "NULL energy");
  if (n_nodes == 0) {
    *energy_host = 0.0;
    return XNN_OK;
  }
  XNN_REQUIRE(pos && atomic_numbers && node_energy && forces, "NULL input or output");
  XNN_REQUIRE(n_edges == 0 || edge_index, "NULL edge_index");
  const PairWs w = pair_layout(n_nodes, n_edges);
  XNN_REQUIRE(workspace && workspace_bytes >= w.total,
              "workspace of %zu bytes needed (xnn_sh_pair_workspace_bytes)", w.total);
  const hipStream_t s = as_hip(stream);
  int32_t* src = at<int32_t>(workspace, w.src);
  int32_t* dst = at<int32_t>(workspace, w.dst);
  int32_t* shift = at<int32_t>(workspace, w.shift);
  int32_t* ptr_dst = at<int32_t>(workspace, w.ptr_dst);
  int32_t* perm_dst = at<int32_t>(workspace, w.perm_dst);
  int32_t* ptr_src = at<int32_t>(workspace, w.ptr_src);
  int32_t* perm_src = at<int32_t>(workspace, w.perm_src);
  int32_t* flag = at<int32_t>(workspace, w.flag);
  int32_t* batch = at<int32_t>(workspace, w.batch);
  float* one = at<float>(workspace, w.one);
  int64_t* seg_ptr = at<int64_t>(workspace, w.seg_ptr);
  float* g_vec = at<float>(workspace, w.g_vec);
  float* vec = at<float>(workspace, w.vec);
  double* partial = at<double>(workspace, w.partial);
  double* energy = at<double>(workspace, w.energy);
  const void* cl = cell;  // NULL: a molecule

  hipLaunchKernelGGL(pair_fill_kernel, dim3((unsigned)grid_1d(n_nodes, 256)), dim3(256), 0, s,
                     batch, n_nodes, one, seg_ptr);
  XNN_LAUNCH_CHECK();
  int rc = xnn_edge_plan(edge_index, cell_shifts, n_edges, n_nodes, src, dst, shift, ptr_dst,
                         perm_dst, ptr_src, perm_src, flag, at<char>(workspace, w.plan),
                         w.plan_bytes, stream);
  if (rc != XNN_OK) return rc;
  const xnn_sh_pair_model& M = *model;
  rc = xnn_sh_radial_message_energy(geom_dtype, nullptr, pos, n_nodes, cl, 1, batch, src, shift,
                                    n_edges, ptr_dst, perm_dst, M.prm, M.rbf_table, M.n_channels,
                                    M.W, M.U, atomic_numbers, M.atom_ref, M.n_atom_ref,
                                    node_energy, stream);
  if (rc != XNN_OK) return rc;
  rc = xnn_sh_radial_message_energy_backward(geom_dtype, nullptr, pos, n_nodes, cl, 1, batch, src,
                                             shift, n_edges, ptr_dst, perm_dst, M.prm,
                                             M.rbf_table, M.n_channels, M.W, M.U, one, 0, g_vec,
                                             stream);
  if (rc != XNN_OK) return rc;
  double* vir_partial = virial ? partial : nullptr;
  if (virial) {
    rc = xnn_edge_featurize(geom_dtype, XNN_F32, nullptr, pos, n_nodes, cl, 1, batch, src, dst,
                            shift, n_edges, M.prm, M.rbf_table, vec, nullptr, nullptr, nullptr,
                            stream);
    if (rc != XNN_OK) return rc;
  }
  rc = xnn_edge_force_reduce(geom_dtype, XNN_F32, g_vec, n_edges, ptr_dst, perm_dst, ptr_src,
                             perm_src, shift, nullptr, n_nodes, forces, nullptr,
                             virial ? vec : nullptr, vir_partial, stream);
  if (rc != XNN_OK) return rc;
  rc = xnn_segment_reduce_f64(XNN_F32, node_energy, n_nodes, 1, seg_ptr, 1, energy,
                              w.seg_bytes ? at<char>(workspace, w.seg) : nullptr, w.seg_bytes,
                              stream);
  if (rc != XNN_OK) return rc;
  if (virial) {
    rc = xnn_virial_reduce(XNN_F64, partial, n_nodes, seg_ptr, 1, nullptr, 1, virial,
                           at<char>(workspace, w.vir), w.vir_bytes, stream);
    if (rc != XNN_OK) return rc;
  }
  if (geom_dtype == XNN_F64)
    hipLaunchKernelGGL(pair_finish_kernel<double>, dim3((unsigned)grid_1d(3 * n_nodes, 256)),
                       dim3(256), 0, s, static_cast<double*>(forces), 3 * n_nodes, virial);
  else
    hipLaunchKernelGGL(pair_finish_kernel<float>, dim3((unsigned)grid_1d(3 * n_nodes, 256)),
                       dim3(256), 0, s, static_cast<float*>(forces), 3 * n_nodes, virial);
  XNN_LAUNCH_CHECK();
  // the step's results are only meaningful for a valid neighbor list: read the plan's flag
  // (and the total energy) back, which ends the call with the stream drained
  int32_t flag_host = 0;
  XNN_HIP_CHECK(hipMemcpyAsync(&flag_host, flag, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  XNN_HIP_CHECK(hipMemcpyAsync(energy_host, energy, sizeof(double), hipMemcpyDeviceToHost, s));
  XNN_HIP_CHECK(hipStreamSynchronize(s));
  XNN_REQUIRE((flag_host & 2) == 0, "edge_index holds atom indices outside [0, %lld)",
              (long long)n_nodes);
  if (flag_host & 1) {
    set_error("cell_shifts outside [-512, 511]");
    return XNN_ECAPACITY;
  }
  return XNN_OK;
}

}  // extern "C"
