// Per-edge featurization, its backward, and the deterministic edge -> atom
// force reduction (gfx950).
//
// xnn_edge_featurize           AtomicGraph.edge_vectors (atomic_data.py:371-418) +
//                              SphericalHarmonicEdgeEmbedding.embed (spherical.py:115-138)
// xnn_edge_featurize_backward  the autograd chain of the above back to r_e
// xnn_edge_force_reduce        _EdgeVectors.backward (atomic_data.py:452-467) without atomics
#include <string.h>

#include <algorithm>

#include "common.h"
#include "device.h"
#include "message.h"

namespace xnn {

thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

template <typename G>
__device__ inline const G* cell_of(const G* cell, int64_t n_graphs, const int32_t* batch,
                                   int node) {
  if (cell == nullptr) return nullptr;
  if (n_graphs <= 1 || batch == nullptr) return cell;
  return cell + 9 * (int64_t)batch[node];
}

// ---------------------------------------------------------------- featurize
// edge vector in the compute dtype: given, or formed from positions
template <typename G, typename T>
__device__ inline void load_edge(const T* __restrict__ vec_in, const G* __restrict__ pos,
                                 const G* __restrict__ cell, int64_t n_graphs,
                                 const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
                                 const int32_t* __restrict__ dst, const int32_t* __restrict__ shift,
                                 int64_t e, T& x, T& y, T& z) {
  if (vec_in != nullptr) {
    x = vec_in[3 * e + 0];
    y = vec_in[3 * e + 1];
    z = vec_in[3 * e + 2];
    return;
  }
  const int s = src[e], d = dst[e];
  G gx, gy, gz;
  edge_vector(pos, s, d, shift[e], cell_of(cell, n_graphs, batch, d), gx, gy, gz);
  x = (T)gx;
  y = (T)gy;
  z = (T)gz;
}

template <typename G, typename T, int LMAX>
__global__ __launch_bounds__(256) void featurize_fwd_kernel(
    const T* __restrict__ vec_in, const G* __restrict__ pos, const G* __restrict__ cell, int64_t n_graphs,
    const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ dst, const int32_t* __restrict__ shift, int64_t n_edges,
    Radial<T> R, int sign, T* __restrict__ vec, T* __restrict__ length, T* __restrict__ sh,
    T* __restrict__ radial) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_edges) return;
  T x, y, z;
  load_edge(vec_in, pos, cell, n_graphs, batch, src, dst, shift, e, x, y, z);
  if (vec) {
    vec[3 * e + 0] = x;
    vec[3 * e + 1] = y;
    vec[3 * e + 2] = z;
  }
  const T r = dev_sqrt(x * x + y * y + z * z);
  if (length) length[e] = r;
  if (sh) {
    constexpr int L = (LMAX + 1) * (LMAX + 1);
    const T inv = r > T(0) ? T(1) / r : T(0);
    const T sg = (T)sign;
    T Y[L];
    sh_eval<LMAX, T>(sg * x * inv, sg * y * inv, sg * z * inv, Y);
#pragma unroll
    for (int k = 0; k < L; ++k) sh[e * L + k] = Y[k];
  }
  if (radial) {
    const RadialAt<T> a = radial_at(R, r);
    for (int k = 0; k < R.K; ++k) {
      T u, du;
      radial_k<T, false>(R, a, k, u, du);
      radial[e * R.K + k] = u;
    }
  }
}

template <typename G, typename T, int LMAX>
__global__ __launch_bounds__(256) void featurize_bwd_kernel(
    const T* __restrict__ vec_in, const G* __restrict__ pos, const G* __restrict__ cell, int64_t n_graphs,
    const int32_t* __restrict__ batch, const int32_t* __restrict__ src,
    const int32_t* __restrict__ dst, const int32_t* __restrict__ shift, int64_t n_edges,
    Radial<T> R, int sign, const T* __restrict__ d_vec, const T* __restrict__ d_length,
    const T* __restrict__ d_sh, const T* __restrict__ d_radial, const T* __restrict__ g_extra,
    T* __restrict__ g_edge) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_edges) return;
  T x, y, z;
  load_edge(vec_in, pos, cell, n_graphs, batch, src, dst, shift, e, x, y, z);
  const T r = dev_sqrt(x * x + y * y + z * z);
  const T inv = r > T(0) ? T(1) / r : T(0);
  const T ux = x * inv, uy = y * inv, uz = z * inv;
  T ox = T(0), oy = T(0), oz = T(0);
  if (d_vec) {
    ox = d_vec[3 * e + 0];
    oy = d_vec[3 * e + 1];
    oz = d_vec[3 * e + 2];
  }
  if (g_extra) {
    ox += g_extra[3 * e + 0];
    oy += g_extra[3 * e + 1];
    oz += g_extra[3 * e + 2];
  }
  T dl = d_length ? d_length[e] : T(0);
  if (d_radial) {
    const RadialAt<T> a = radial_at(R, r);
    for (int k = 0; k < R.K; ++k) {
      T u, du;
      radial_k<T, true>(R, a, k, u, du);
      dl += d_radial[e * R.K + k] * du;
    }
  }
  ox += dl * ux;
  oy += dl * uy;
  oz += dl * uz;
  if (d_sh && r > T(0)) {
    constexpr int L = (LMAX + 1) * (LMAX + 1);
    T dY[L];
#pragma unroll
    for (int k = 0; k < L; ++k) dY[k] = d_sh[e * L + k];
    const T sg = (T)sign;
    T Gx, Gy, Gz, vx, vy, vz;
    sh_grad<LMAX, T>(sg * ux, sg * uy, sg * uz, dY, Gx, Gy, Gz);
    sh_chain<T>(sg * ux, sg * uy, sg * uz, inv, Gx, Gy, Gz, vx, vy, vz);
    ox += sg * vx;
    oy += sg * vy;
    oz += sg * vz;
  }
  g_edge[3 * e + 0] = ox;
  g_edge[3 * e + 1] = oy;
  g_edge[3 * e + 2] = oz;
}

// ---------------------------------------------------------------- force reduce
// GROUP lanes per atom: lanes stride over the atom's receiver and sender rows,
// then a fixed butterfly sums the lanes (bitwise reproducible).
//
// Atoms are taken in the order `visit` (NULL: index order), a spatial order of the atoms
// (the plan's space-filling curve), and the blocks are laid out over the XCDs: workgroups
// are dispatched to the 8 XCDs in turn, so block b is given slot block
// (b % 8) * per_xcd + b / 8 and each XCD walks one contiguous run of the visit order. The
// sender-side gather of an atom reads the gradient rows of its neighbours; with spatially
// compact runs those rows are shared by the XCD's other atoms and stay in its L2.

template <typename G, typename T, int GROUP>
__global__ __launch_bounds__(256) void force_reduce_kernel(
    const T* __restrict__ g_edge, const int32_t* __restrict__ ptr_dst,
    const int32_t* __restrict__ perm_dst, const int32_t* __restrict__ ptr_src,
    const int32_t* __restrict__ perm_src, const int32_t* __restrict__ shift,
    const int32_t* __restrict__ visit, int64_t n_nodes, G* __restrict__ grad_pos,
    double* __restrict__ cell_partial, const T* __restrict__ vec,
    double* __restrict__ virial_partial, double* __restrict__ virial_block) {
  const int lane = threadIdx.x % GROUP;
  const int64_t sb = xcd_slot();
  const int64_t slot = (sb * blockDim.x + threadIdx.x) / GROUP;
  const bool live = slot < n_nodes;
  const int64_t i = live ? (visit ? (int64_t)visit[slot] : slot) : 0;
  const bool want_cell = cell_partial != nullptr;
  const bool want_vir = virial_partial != nullptr || virial_block != nullptr;
  double fx = 0, fy = 0, fz = 0;
  double c[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  double v[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  if (live) {
    const int b0 = ptr_dst[i], b1 = ptr_dst[i + 1];
    for (int k = b0 + lane; k < b1; k += GROUP) {
      const int e = perm_dst ? perm_dst[k] : k;
      const double x = g_edge[3 * (int64_t)e + 0], y = g_edge[3 * (int64_t)e + 1],
                   z = g_edge[3 * (int64_t)e + 2];
      fx += x;
      fy += y;
      fz += z;
      if (want_cell) {
        int sx, sy, sz;
        unpack_shift(shift[e], sx, sy, sz);
        c[0] += sx * x; c[1] += sx * y; c[2] += sx * z;
        c[3] += sy * x; c[4] += sy * y; c[5] += sy * z;
        c[6] += sz * x; c[7] += sz * y; c[8] += sz * z;
      }
      if (want_vir) {
        const double rx = vec[3 * (int64_t)e + 0], ry = vec[3 * (int64_t)e + 1],
                     rz = vec[3 * (int64_t)e + 2];
        v[0] += rx * x; v[1] += rx * y; v[2] += rx * z;
        v[3] += ry * x; v[4] += ry * y; v[5] += ry * z;
        v[6] += rz * x; v[7] += rz * y; v[8] += rz * z;
      }
    }
    const int s0 = ptr_src[i], s1 = ptr_src[i + 1];
    for (int k = s0 + lane; k < s1; k += GROUP) {
      const int e = perm_src ? perm_src[k] : k;
      fx -= g_edge[3 * (int64_t)e + 0];
      fy -= g_edge[3 * (int64_t)e + 1];
      fz -= g_edge[3 * (int64_t)e + 2];
    }
  }
  // the group's sums in every lane (the butterfly of __shfl_xor, on VALU exchanges)
  fx = group_sum<GROUP>(fx);
  fy = group_sum<GROUP>(fy);
  fz = group_sum<GROUP>(fz);
  if (want_cell) {
#pragma unroll
    for (int q = 0; q < 9; ++q) c[q] = group_sum<GROUP>(c[q]);
  }
  if (want_vir) {
#pragma unroll
    for (int q = 0; q < 9; ++q) v[q] = group_sum<GROUP>(v[q]);
  }
  if (live && lane == 0) {
    grad_pos[3 * i + 0] = (G)fx;
    grad_pos[3 * i + 1] = (G)fy;
    grad_pos[3 * i + 2] = (G)fz;
    if (cell_partial) {
#pragma unroll
      for (int q = 0; q < 9; ++q) cell_partial[9 * i + q] = c[q];
    }
    if (virial_partial) {
#pragma unroll
      for (int q = 0; q < 9; ++q) virial_partial[9 * i + q] = v[q];
    }
  }
  if (virial_block != nullptr) {
    // the block's atoms' r (x) g summed in group order (one structure)
    __shared__ double gsum[256 / GROUP][9];
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 9; ++q) gsum[threadIdx.x / GROUP][q] = live ? v[q] : 0.0;
    }
    __syncthreads();
    if (threadIdx.x < 9) {
      double a = 0.0;
      for (int g = 0; g < 256 / GROUP; ++g) a += gsum[g][threadIdx.x];
      virial_block[9 * (int64_t)blockIdx.x + threadIdx.x] = a;
    }
  }
}

// One block: out (3,3) = sym(sum_b block[b]) with the rows taken in a fixed order (thread t
// sums rows t, t + 256, ...; then each wave's butterfly and the 4 wave sums in order).
template <typename OUT>
__global__ __launch_bounds__(256) void virial_blocks_finish_kernel(const double* __restrict__ block,
                                                                   int64_t n_blocks,
                                                                   OUT* __restrict__ out) {
  double a[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t b = threadIdx.x; b < n_blocks; b += 256) {
#pragma unroll
    for (int q = 0; q < 9; ++q) a[q] += block[9 * b + q];
  }
#pragma unroll
  for (int q = 0; q < 9; ++q) a[q] = group_sum<kWave>(a[q]);
  __shared__ double wsum[256 / kWave][9];
  __shared__ double tot[9];
  if (threadIdx.x % kWave == 0) {
#pragma unroll
    for (int q = 0; q < 9; ++q) wsum[threadIdx.x / kWave][q] = a[q];
  }
  __syncthreads();
  if (threadIdx.x < 9) {
    double t = 0.0;
    for (int w = 0; w < 256 / kWave; ++w) t += wsum[w][threadIdx.x];
    tot[threadIdx.x] = t;
  }
  __syncthreads();
  if (threadIdx.x < 9) {
    const int r = threadIdx.x / 3, c = threadIdx.x % 3;
    out[threadIdx.x] = (OUT)(0.5 * (tot[threadIdx.x] + tot[3 * c + r]));
  }
}

// ---------------------------------------------------------------- strain deformation
// S_b = (eps_b + eps_b^T) / 2; pos'_i = pos_i (I + S_b), cell'_b = cell_b (I + S_b)
// (outputs.py:166-180). Row vectors: (x S)_k = sum_j x_j S_jk.
template <typename G>
__device__ inline void sym_of(const G* __restrict__ eps, int64_t b, double S[9]) {
  const G* e = eps + 9 * b;
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int k = 0; k < 3; ++k) S[3 * j + k] = 0.5 * ((double)e[3 * j + k] + (double)e[3 * k + j]);
}

template <typename G>
__global__ __launch_bounds__(256) void strain_fwd_kernel(
    const G* __restrict__ pos, int64_t n_nodes, const int32_t* __restrict__ batch,
    const G* __restrict__ cell, int64_t n_graphs, const G* __restrict__ eps,
    G* __restrict__ pos_out, G* __restrict__ cell_out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n_nodes) {
    double S[9];
    sym_of(eps, batch ? batch[t] : 0, S);
    const G x = pos[3 * t], y = pos[3 * t + 1], z = pos[3 * t + 2];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      pos_out[3 * t + k] = pos[3 * t + k] + (G)(x * S[k] + y * S[3 + k] + z * S[6 + k]);
  }
  if (cell != nullptr && t < 3 * n_graphs) {   // one cell row per thread
    const int64_t b = t / 3;
    double S[9];
    sym_of(eps, b, S);
    const G* r = cell + 3 * t;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      cell_out[3 * t + k] = r[k] + (G)(r[0] * S[k] + r[1] * S[3 + k] + r[2] * S[6 + k]);
  }
}

// grad_pos_i = g_i (I + S_b)^T; partial_i = pos_i (x) g_i (float64, to be summed per
// structure); grad_cell_b = g_cell_b (I + S_b)^T; cell_term_b = cell_b^T g_cell_b.
template <typename G>
__global__ __launch_bounds__(256) void strain_bwd_kernel(
    const G* __restrict__ pos, int64_t n_nodes, const int32_t* __restrict__ batch,
    const G* __restrict__ cell, int64_t n_graphs, const G* __restrict__ eps,
    const G* __restrict__ g_pos, const G* __restrict__ g_cell, G* __restrict__ grad_pos,
    G* __restrict__ grad_cell, double* __restrict__ partial, double* __restrict__ cell_term) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n_nodes) {
    double S[9];
    sym_of(eps, batch ? batch[t] : 0, S);
    const double gx = g_pos[3 * t], gy = g_pos[3 * t + 1], gz = g_pos[3 * t + 2];
    // (g S^T)_j = sum_k g_k S_jk
#pragma unroll
    for (int j = 0; j < 3; ++j)
      grad_pos[3 * t + j] = (G)((double)g_pos[3 * t + j] + gx * S[3 * j] + gy * S[3 * j + 1] +
                                gz * S[3 * j + 2]);
    const double x = pos[3 * t], y = pos[3 * t + 1], z = pos[3 * t + 2];
    double* m = partial + 9 * t;
    m[0] = x * gx; m[1] = x * gy; m[2] = x * gz;
    m[3] = y * gx; m[4] = y * gy; m[5] = y * gz;
    m[6] = z * gx; m[7] = z * gy; m[8] = z * gz;
  }
  if (cell != nullptr && t < n_graphs) {
    double S[9];
    sym_of(eps, t, S);
    const G* c = cell + 9 * t;
    const G* gc = g_cell + 9 * t;
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        double v = gc[3 * a + j];
#pragma unroll
        for (int k = 0; k < 3; ++k) v += (double)gc[3 * a + k] * S[3 * j + k];
        grad_cell[9 * t + 3 * a + j] = (G)v;
      }
    // (cell^T g)_jk = sum_a cell_aj g_ak
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        double v = 0.0;
#pragma unroll
        for (int a = 0; a < 3; ++a) v += (double)c[3 * a + j] * (double)gc[3 * a + k];
        cell_term[9 * t + 3 * j + k] = v;
      }
  }
}

// out[b] = sym(M[b] + term[b]) (or unsymmetrized), float64 in, dtype out
template <typename T>
__global__ __launch_bounds__(256) void virial_finish_kernel(const double* __restrict__ M,
                                                            const double* __restrict__ term,
                                                            int64_t n_graphs, int symmetrize,
                                                            T* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 9 * n_graphs) return;
  const int64_t b = t / 9;
  const int j = (int)(t - 9 * b), r = j / 3, c = j % 3;
  double v = M[t] + (term ? term[t] : 0.0);
  if (symmetrize) {
    const int64_t u = 9 * b + 3 * c + r;
    v = 0.5 * (v + M[u] + (term ? term[u] : 0.0));
  }
  out[t] = (T)v;
}

// stress[b] = scale g[b] / V_b for periodic structures, V_b = |det cell_b| > 1e-8 and (with
// pbc) some periodic direction; zero otherwise (outputs.py:227-239). float64 inside.
template <typename T, typename C>
__global__ __launch_bounds__(256) void stress_finish_kernel(const T* __restrict__ g,
                                                            const C* __restrict__ cell,
                                                            const uint8_t* __restrict__ pbc,
                                                            int64_t n_graphs, double scale,
                                                            T* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 9 * n_graphs) return;
  out[t] = stress_entry(g, cell, pbc, t / 9, (int)(t % 9), scale);
}

// ---------------------------------------------------------------- dispatch helpers

template <typename G, typename T>
static int featurize_fwd(const void* vec_in, const void* pos, const void* cell, int64_t n_graphs,
                         const int32_t* batch, const int32_t* src, const int32_t* dst,
                         const int32_t* shift, int64_t n_edges,
                         const xnn_featurize_params* prm, const void* table, void* vec,
                         void* length, void* sh, void* radial, hipStream_t stream) {
  Radial<T> R;
  int st = make_radial<T>(prm, table, R);
  if (st != XNN_OK) return st;
  if (n_edges == 0) return XNN_OK;
  const dim3 grid(grid_1d(n_edges, 256)), block(256);
#define XNN_FWD(LM)                                                                      \
  hipLaunchKernelGGL((featurize_fwd_kernel<G, T, LM>), grid, block, 0, stream,           \
                     (const T*)vec_in, (const G*)pos, (const G*)cell, n_graphs, batch, src, dst, shift,    \
                     n_edges, R, prm->sh_sign, (T*)vec, (T*)length, (T*)sh, (T*)radial)
  switch (prm->l_max) {
    case 0: XNN_FWD(0); break;
    case 1: XNN_FWD(1); break;
    case 2: XNN_FWD(2); break;
    default: XNN_FWD(3); break;
  }
#undef XNN_FWD
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

template <typename G, typename T>
static int featurize_bwd(const void* vec_in, const void* pos, const void* cell, int64_t n_graphs,
                         const int32_t* batch, const int32_t* src, const int32_t* dst,
                         const int32_t* shift, int64_t n_edges,
                         const xnn_featurize_params* prm, const void* table, const void* d_vec,
                         const void* d_length, const void* d_sh, const void* d_radial,
                         const void* g_extra, void* g_edge, hipStream_t stream) {
  Radial<T> R;
  int st = make_radial<T>(prm, table, R);
  if (st != XNN_OK) return st;
  if (n_edges == 0) return XNN_OK;
  const dim3 grid(grid_1d(n_edges, 256)), block(256);
#define XNN_BWD(LM)                                                                       \
  hipLaunchKernelGGL((featurize_bwd_kernel<G, T, LM>), grid, block, 0, stream,            \
                     (const T*)vec_in, (const G*)pos, (const G*)cell, n_graphs, batch, src, dst, shift,     \
                     n_edges, R, prm->sh_sign, (const T*)d_vec, (const T*)d_length,       \
                     (const T*)d_sh, (const T*)d_radial, (const T*)g_extra, (T*)g_edge)
  switch (prm->l_max) {
    case 0: XNN_BWD(0); break;
    case 1: XNN_BWD(1); break;
    case 2: XNN_BWD(2); break;
    default: XNN_BWD(3); break;
  }
#undef XNN_BWD
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

// lanes per atom from the mean degree (both rows are walked)
static int force_group(int64_t n_edges, int64_t n_nodes) {
  const double deg = n_nodes > 0 ? (double)n_edges / (double)n_nodes : 0.0;
  return deg > 24 ? 32 : (deg > 6 ? 16 : 4);
}

// blocks of the force reduction: enough for every atom, rounded up to whole XCD rounds
static int64_t force_blocks(int64_t n_edges, int64_t n_nodes) {
  return xcd_blocks(grid_1d(n_nodes * force_group(n_edges, n_nodes), 256));
}

template <typename G, typename T, int GROUP>
static void launch_force_reduce(int64_t n_blocks, const void* g_edge, const int32_t* ptr_dst,
                                const int32_t* perm_dst, const int32_t* ptr_src,
                                const int32_t* perm_src, const int32_t* shift,
                                const int32_t* visit, int64_t n_nodes, void* grad_pos,
                                double* cell_partial, const void* vec, double* virial_partial,
                                double* virial_block, hipStream_t stream) {
  hipLaunchKernelGGL((force_reduce_kernel<G, T, GROUP>), dim3((unsigned)n_blocks), dim3(256), 0,
                     stream, (const T*)g_edge, ptr_dst, perm_dst, ptr_src, perm_src, shift, visit,
                     n_nodes, (G*)grad_pos, cell_partial, (const T*)vec, virial_partial,
                     virial_block);
}

template <typename G, typename T>
static int force_reduce(const void* g_edge, int64_t n_edges, const int32_t* ptr_dst,
                        const int32_t* perm_dst, const int32_t* ptr_src,
                        const int32_t* perm_src, const int32_t* shift, const int32_t* visit,
                        int64_t n_nodes, void* grad_pos, double* cell_partial, const void* vec,
                        double* virial_partial, double* virial_block, hipStream_t stream) {
  if (n_nodes == 0) return XNN_OK;
  const int64_t nb = force_blocks(n_edges, n_nodes);
  switch (force_group(n_edges, n_nodes)) {
    case 32:
      launch_force_reduce<G, T, 32>(nb, g_edge, ptr_dst, perm_dst, ptr_src, perm_src, shift, visit,
                                    n_nodes, grad_pos, cell_partial, vec, virial_partial, virial_block,
                                    stream);
      break;
    case 16:
      launch_force_reduce<G, T, 16>(nb, g_edge, ptr_dst, perm_dst, ptr_src, perm_src, shift, visit,
                                    n_nodes, grad_pos, cell_partial, vec, virial_partial, virial_block,
                                    stream);
      break;
    default:
      launch_force_reduce<G, T, 4>(nb, g_edge, ptr_dst, perm_dst, ptr_src, perm_src, shift, visit,
                                   n_nodes, grad_pos, cell_partial, vec, virial_partial, virial_block,
                                   stream);
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // namespace xnn

using namespace xnn;

#define XNN_DISPATCH_GT(geom, comp, FN, ...)                                         \
  do {                                                                               \
    if ((geom) == XNN_F32 && (comp) == XNN_F32) return FN<float, float>(__VA_ARGS__); \
    if ((geom) == XNN_F64 && (comp) == XNN_F64)                                      \
      return FN<double, double>(__VA_ARGS__);                                        \
    if ((geom) == XNN_F64 && (comp) == XNN_F32)                                      \
      return FN<double, float>(__VA_ARGS__);                                         \
    set_error("unsupported dtype pair geometry=%d compute=%d", (int)(geom), (int)(comp)); \
    return XNN_EINVAL;                                                               \
  } while (0)

extern "C" {

const char* xnn_last_error(void) { return g_error; }
int xnn_abi_version(void) { return 2; }

int xnn_edge_featurize(int geom_dtype, int compute_dtype, const void* vec_in, const void* pos,
                       int64_t n_nodes, const void* cell, int64_t n_graphs, const int32_t* batch,
                       const int32_t* src, const int32_t* dst, const int32_t* shift,
                       int64_t n_edges, const xnn_featurize_params* prm, const void* rbf_table,
                       void* vec, void* length, void* sh, void* radial, xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_nodes >= 0, "negative size");
  XNN_REQUIRE(n_edges == 0 || vec_in || (pos && src && dst && shift), "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  XNN_DISPATCH_GT(geom_dtype, compute_dtype, featurize_fwd, vec_in, pos, cell, n_graphs, batch, src,
                  dst, shift, n_edges, prm, rbf_table, vec, length, sh, radial,
                  as_hip(stream));
}

int xnn_edge_featurize_backward(int geom_dtype, int compute_dtype, const void* vec_in,
                                const void* pos, int64_t n_nodes, const void* cell, int64_t n_graphs,
                                const int32_t* batch, const int32_t* src, const int32_t* dst,
                                const int32_t* shift, int64_t n_edges,
                                const xnn_featurize_params* prm, const void* rbf_table,
                                const void* d_vec, const void* d_length, const void* d_sh,
                                const void* d_radial, const void* g_extra, void* g_edge,
                                xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_nodes >= 0, "negative size");
  XNN_REQUIRE(n_edges == 0 || ((vec_in || (pos && src && dst && shift)) && g_edge),
              "NULL edge input");
  XNN_REQUIRE(cell == nullptr || n_graphs <= 1 || batch != nullptr,
              "several cells need the batch vector");
  XNN_DISPATCH_GT(geom_dtype, compute_dtype, featurize_bwd, vec_in, pos, cell, n_graphs, batch, src,
                  dst, shift, n_edges, prm, rbf_table, d_vec, d_length, d_sh, d_radial,
                  g_extra, g_edge, as_hip(stream));
}

int xnn_edge_force_reduce(int geom_dtype, int compute_dtype, const void* g_edge, int64_t n_edges,
                          const int32_t* ptr_dst, const int32_t* perm_dst,
                          const int32_t* ptr_src, const int32_t* perm_src,
                          const int32_t* shift, const int32_t* visit, int64_t n_nodes,
                          void* grad_pos, double* cell_partial, const void* vec,
                          double* virial_partial, xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_nodes >= 0, "negative size");
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && ptr_src && grad_pos), "NULL CSR or output");
  XNN_REQUIRE(n_edges == 0 || g_edge, "NULL g_edge");
  XNN_REQUIRE(cell_partial == nullptr || shift != nullptr, "cell_partial needs the shifts");
  XNN_REQUIRE(virial_partial == nullptr || n_edges == 0 || vec != nullptr,
              "virial_partial needs the edge vectors");
  XNN_DISPATCH_GT(geom_dtype, compute_dtype, force_reduce, g_edge, n_edges, ptr_dst, perm_dst,
                  ptr_src, perm_src, shift, visit, n_nodes, grad_pos, cell_partial, vec,
                  virial_partial, nullptr, as_hip(stream));
}

size_t xnn_edge_force_reduce_virial_workspace_bytes(int64_t n_edges, int64_t n_nodes) {
  if (n_edges < 0 || n_nodes <= 0) return 0;
  return sizeof(double) * 9 * (size_t)force_blocks(n_edges, n_nodes);
}

int xnn_edge_force_reduce_virial(int geom_dtype, int compute_dtype, const void* g_edge,
                                 int64_t n_edges, const int32_t* ptr_dst, const int32_t* perm_dst,
                                 const int32_t* ptr_src, const int32_t* perm_src,
                                 const int32_t* visit, int64_t n_nodes, void* grad_pos,
                                 const void* vec, int virial_dtype, void* virial,
                                 void* workspace, size_t workspace_bytes, xnn_stream_t stream) {
  XNN_REQUIRE(n_edges >= 0 && n_nodes >= 0, "negative size");
  XNN_REQUIRE(virial != nullptr, "NULL virial");
  XNN_REQUIRE(virial_dtype == XNN_F32 || virial_dtype == XNN_F64,
              "virial dtype must be XNN_F32 or XNN_F64");
  XNN_REQUIRE(n_nodes == 0 || (ptr_dst && ptr_src && grad_pos), "NULL CSR or output");
  XNN_REQUIRE(n_edges == 0 || (g_edge && vec), "NULL g_edge or edge vectors");
  const size_t need = xnn_edge_force_reduce_virial_workspace_bytes(n_edges, n_nodes);
  XNN_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
              "workspace of %zu bytes needed", need);
  double* block = static_cast<double*>(workspace);
  const int64_t nb = n_nodes > 0 ? force_blocks(n_edges, n_nodes) : 0;
  hipStream_t st = as_hip(stream);
  if (n_nodes > 0) {
    int rc = XNN_OK;
    if (geom_dtype == XNN_F32 && compute_dtype == XNN_F32)
      rc = force_reduce<float, float>(g_edge, n_edges, ptr_dst, perm_dst, ptr_src, perm_src,
                                      nullptr, visit, n_nodes, grad_pos, nullptr, vec, nullptr,
                                      block, st);
    else if (geom_dtype == XNN_F64 && compute_dtype == XNN_F64)
      rc = force_reduce<double, double>(g_edge, n_edges, ptr_dst, perm_dst, ptr_src, perm_src,
                                        nullptr, visit, n_nodes, grad_pos, nullptr, vec, nullptr,
                                        block, st);
    else if (geom_dtype == XNN_F64 && compute_dtype == XNN_F32)
      rc = force_reduce<double, float>(g_edge, n_edges, ptr_dst, perm_dst, ptr_src, perm_src,
                                       nullptr, visit, n_nodes, grad_pos, nullptr, vec, nullptr,
                                       block, st);
    else
      XNN_REQUIRE(false, "unsupported dtype pair geometry=%d compute=%d", geom_dtype,
                  compute_dtype);
    if (rc != XNN_OK) return rc;
  }
  if (virial_dtype == XNN_F64)
    hipLaunchKernelGGL(virial_blocks_finish_kernel<double>, dim3(1), dim3(256), 0, st, block, nb,
                       static_cast<double*>(virial));
  else
    hipLaunchKernelGGL(virial_blocks_finish_kernel<float>, dim3(1), dim3(256), 0, st, block, nb,
                       static_cast<float*>(virial));
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_strain_apply(int geom_dtype, const void* pos, int64_t n_nodes, const int32_t* batch,
                     const void* cell, int64_t n_graphs, const void* strain, void* pos_out,
                     void* cell_out, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_graphs >= 1, "bad sizes");
  XNN_REQUIRE(strain != nullptr && (n_nodes == 0 || (pos && pos_out)), "NULL input or output");
  XNN_REQUIRE(n_graphs == 1 || batch != nullptr, "several structures need the batch vector");
  XNN_REQUIRE(cell == nullptr || cell_out != nullptr, "NULL cell_out");
  const int64_t n = std::max<int64_t>(n_nodes, 3 * n_graphs);
  if (n == 0) return XNN_OK;
  hipStream_t s = as_hip(stream);
  if (geom_dtype == XNN_F32)
    hipLaunchKernelGGL(strain_fwd_kernel<float>, dim3(grid_1d(n, 256)), dim3(256), 0, s,
                       (const float*)pos, n_nodes, batch, (const float*)cell, n_graphs,
                       (const float*)strain, (float*)pos_out, (float*)cell_out);
  else if (geom_dtype == XNN_F64)
    hipLaunchKernelGGL(strain_fwd_kernel<double>, dim3(grid_1d(n, 256)), dim3(256), 0, s,
                       (const double*)pos, n_nodes, batch, (const double*)cell, n_graphs,
                       (const double*)strain, (double*)pos_out, (double*)cell_out);
  else {
    set_error("unsupported geometry dtype %d", geom_dtype);
    return XNN_EINVAL;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_strain_apply_backward(int geom_dtype, const void* pos, int64_t n_nodes,
                              const int32_t* batch, const void* cell, int64_t n_graphs,
                              const void* strain, const void* g_pos, const void* g_cell,
                              void* grad_pos, void* grad_cell, double* partial,
                              double* cell_term, xnn_stream_t stream) {
  XNN_REQUIRE(n_nodes >= 0 && n_graphs >= 1, "bad sizes");
  XNN_REQUIRE(strain != nullptr && (n_nodes == 0 || (pos && g_pos && grad_pos && partial)),
              "NULL input or output");
  XNN_REQUIRE(n_graphs == 1 || batch != nullptr, "several structures need the batch vector");
  XNN_REQUIRE(cell == nullptr || (g_cell && grad_cell && cell_term), "NULL cell gradient");
  const int64_t n = std::max<int64_t>(n_nodes, n_graphs);
  if (n == 0) return XNN_OK;
  hipStream_t s = as_hip(stream);
  if (geom_dtype == XNN_F32)
    hipLaunchKernelGGL(strain_bwd_kernel<float>, dim3(grid_1d(n, 256)), dim3(256), 0, s,
                       (const float*)pos, n_nodes, batch, (const float*)cell, n_graphs,
                       (const float*)strain, (const float*)g_pos, (const float*)g_cell,
                       (float*)grad_pos, (float*)grad_cell, partial, cell_term);
  else if (geom_dtype == XNN_F64)
    hipLaunchKernelGGL(strain_bwd_kernel<double>, dim3(grid_1d(n, 256)), dim3(256), 0, s,
                       (const double*)pos, n_nodes, batch, (const double*)cell, n_graphs,
                       (const double*)strain, (const double*)g_pos, (const double*)g_cell,
                       (double*)grad_pos, (double*)grad_cell, partial, cell_term);
  else {
    set_error("unsupported geometry dtype %d", geom_dtype);
    return XNN_EINVAL;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_stress_finish(int dtype, const void* strain_grad, int cell_dtype, const void* cell,
                      const uint8_t* pbc, int64_t n_graphs, double scale, void* stress,
                      xnn_stream_t stream) {
  XNN_REQUIRE(n_graphs >= 0, "negative size");
  if (n_graphs == 0) return XNN_OK;
  XNN_REQUIRE(strain_grad && cell && stress, "NULL input or output");
  hipStream_t s = as_hip(stream);
  const dim3 grid(grid_1d(9 * n_graphs, 256)), block(256);
#define XNN_SF(T, C)                                                                     \
  hipLaunchKernelGGL((stress_finish_kernel<T, C>), grid, block, 0, s, (const T*)strain_grad, \
                     (const C*)cell, pbc, n_graphs, scale, (T*)stress)
  if (dtype == XNN_F32 && cell_dtype == XNN_F32) XNN_SF(float, float);
  else if (dtype == XNN_F32 && cell_dtype == XNN_F64) XNN_SF(float, double);
  else if (dtype == XNN_F64 && cell_dtype == XNN_F32) XNN_SF(double, float);
  else if (dtype == XNN_F64 && cell_dtype == XNN_F64) XNN_SF(double, double);
  else {
    set_error("unsupported dtypes %d / %d", dtype, cell_dtype);
    return XNN_EINVAL;
  }
#undef XNN_SF
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

int xnn_virial_finish(int dtype, const double* M, const double* term, int64_t n_graphs,
                      int32_t symmetrize, void* out, xnn_stream_t stream) {
  XNN_REQUIRE(n_graphs >= 0, "negative size");
  if (n_graphs == 0) return XNN_OK;
  XNN_REQUIRE(M && out, "NULL input or output");
  hipStream_t s = as_hip(stream);
  const dim3 grid(grid_1d(9 * n_graphs, 256)), block(256);
  if (dtype == XNN_F32)
    hipLaunchKernelGGL(virial_finish_kernel<float>, grid, block, 0, s, M, term, n_graphs,
                       (int)symmetrize, (float*)out);
  else if (dtype == XNN_F64)
    hipLaunchKernelGGL(virial_finish_kernel<double>, grid, block, 0, s, M, term, n_graphs,
                       (int)symmetrize, (double*)out);
  else {
    set_error("unsupported dtype %d", dtype);
    return XNN_EINVAL;
  }
  XNN_LAUNCH_CHECK();
  return XNN_OK;
}

}  // extern "C"
