// Host-side checks of the C ABI under AddressSanitizer: the entry points that run on the
// host only (plans, workspace sizes, argument validation and the error text) are called
// with ordinary, edge-case and invalid arguments. No GPU is needed: every call here returns
// before any HIP launch. Built by tests/test_host_asan.py with the host pass of every
// library source instrumented; a memory error aborts with ASan's report.
#include <cmath>
#include <cstdio>
#include <cstring>

#include "xnn_amd.h"

static int failures = 0;

#define CHECK(cond)                                                          \
  do {                                                                       \
    if (!(cond)) {                                                           \
      std::printf("FAILED %s:%d: %s (%s)\n", __FILE__, __LINE__, #cond,     \
                  xnn_last_error());                                         \
      ++failures;                                                            \
    }                                                                        \
  } while (0)

static void plans() {
  xnn_grid_plan plan;
  const int32_t none[3] = {0, 0, 0}, all[3] = {1, 1, 1}, slab[3] = {1, 1, 0};
  const double lo[3] = {-3.0, -2.0, -1.0}, hi[3] = {7.0, 5.0, 9.0};
  // a molecule: Cartesian grid over the coordinate range
  CHECK(xnn_radius_graph_plan(100, nullptr, none, 5.0, lo, hi, &plan) == XNN_OK);
  CHECK(plan.has_cell == 0 && plan.n_bins >= 1 && plan.workspace_bytes > 0);
  // cubic, triclinic and slab cells; a cell far larger than the cutoff
  const double cubic[9] = {20, 0, 0, 0, 20, 0, 0, 0, 20};
  const double tri[9] = {12, 0, 0, 4, 11, 0, 2, 3, 13};
  const double big[9] = {500, 0, 0, 0, 500, 0, 0, 0, 500};
  const double flo[3] = {0.0, 0.0, -0.2}, fhi[3] = {1.0, 1.0, 1.3};
  CHECK(xnn_radius_graph_plan(9000, cubic, all, 5.0, flo, fhi, &plan) == XNN_OK);
  CHECK(plan.has_cell == 1 && plan.nbins[0] >= 1 && plan.n_bins == (int64_t)plan.nbins[0] * plan.nbins[1] * plan.nbins[2]);
  CHECK(xnn_radius_graph_plan(500, tri, all, 6.0, flo, fhi, &plan) == XNN_OK);
  CHECK(xnn_radius_graph_plan(800, tri, slab, 6.0, flo, fhi, &plan) == XNN_OK);
  CHECK(xnn_radius_graph_plan(1000000, big, all, 2.0, flo, fhi, &plan) == XNN_OK);
  CHECK(plan.workspace_bytes > 0);
  CHECK(xnn_radius_graph_plan(0, cubic, all, 5.0, flo, fhi, &plan) == XNN_OK);
  // invalid: no plan, no pbc, a cutoff that is not positive or not finite, too many atoms
  CHECK(xnn_radius_graph_plan(10, cubic, all, 5.0, flo, fhi, nullptr) == XNN_EINVAL);
  CHECK(std::strlen(xnn_last_error()) > 0);
  CHECK(xnn_radius_graph_plan(10, cubic, nullptr, 5.0, flo, fhi, &plan) == XNN_EINVAL);
  CHECK(xnn_radius_graph_plan(10, cubic, all, -1.0, flo, fhi, &plan) == XNN_EINVAL);
  CHECK(xnn_radius_graph_plan(10, cubic, all, NAN, flo, fhi, &plan) == XNN_EINVAL);
  CHECK(xnn_radius_graph_plan(-1, cubic, all, 5.0, flo, fhi, &plan) == XNN_EINVAL);
  CHECK(xnn_radius_graph_plan(10, nullptr, none, 5.0, nullptr, nullptr, &plan) == XNN_EINVAL);
}

static void workspaces() {
  const int64_t sizes[] = {0, 1, 63, 64, 65, 4000, 9000, 477698, 100000000};
  for (int64_t n : sizes) {
    (void)xnn_edge_force_reduce_virial_workspace_bytes(n * 50, n);
    (void)xnn_sh_pair_workspace_bytes(n, n * 50);
    (void)xnn_virial_reduce_workspace_bytes(n, 1);
    (void)xnn_virial_reduce_workspace_bytes(n, n > 0 ? n / 2 + 1 : 0);
    (void)xnn_segment_reduce_workspace_bytes(n, 1, 1);
    (void)xnn_segment_reduce_workspace_bytes(n, 9, n > 0 ? n : 1);
    (void)xnn_scan_workspace_bytes(n);
    (void)xnn_edge_plan_workspace_bytes(n * 50, n);
    (void)xnn_d4_plan_bytes(n, 1);
    if (n <= 100000) (void)xnn_d4_workspace_bytes(n, 1, n > 0 ? n : 1);
  }
  CHECK(xnn_edge_force_reduce_virial_workspace_bytes(-1, 5) == 0);
  CHECK(xnn_segment_reduce_noalloc_max_bytes() > 0);
  CHECK(xnn_energy_stress_max_nodes() > 0);
}

static void argument_errors() {
  double out[15];
  float virial[9];
  // every call below fails its argument checks before any device work
  CHECK(xnn_radius_graph_status(XNN_F32, 5, nullptr, nullptr, nullptr, nullptr, nullptr) ==
        XNN_EINVAL);
  CHECK(xnn_radius_graph_status(7, 5, nullptr, nullptr, nullptr, nullptr, nullptr) == XNN_EINVAL);
  CHECK(xnn_segment_reduce_f64_noalloc(XNN_F32, nullptr, int64_t(1) << 20, 1024, nullptr, 1,
                                       nullptr, nullptr) == XNN_EINVAL);
  CHECK(xnn_radius_graph_bounds(XNN_F32, nullptr, 10, nullptr, out, nullptr) == XNN_EINVAL);
  CHECK(xnn_radius_graph_bounds(XNN_F32, out, -1, nullptr, out, nullptr) == XNN_EINVAL);
  CHECK(xnn_radius_graph_bounds(XNN_F32, out, 10, nullptr, nullptr, nullptr) == XNN_EINVAL);
  CHECK(xnn_edge_force_reduce_virial(XNN_F32, XNN_F32, nullptr, -1, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, 0, nullptr, nullptr, XNN_F32, virial,
                                     nullptr, 0, nullptr) == XNN_EINVAL);
  CHECK(xnn_edge_force_reduce_virial(XNN_F32, XNN_F32, nullptr, 0, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, 0, nullptr, nullptr, 7, virial, nullptr,
                                     0, nullptr) == XNN_EINVAL);
  CHECK(xnn_edge_force_reduce_virial(XNN_F32, XNN_F32, nullptr, 10, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, 5, nullptr, nullptr, XNN_F32, virial,
                                     nullptr, 0, nullptr) == XNN_EINVAL);
  CHECK(xnn_energy_stress_finish(XNN_F32, nullptr, xnn_energy_stress_max_nodes() + 1, XNN_F32,
                                 virial, XNN_F32, virial, nullptr, 1.0, out, virial,
                                 nullptr) == XNN_EINVAL);
  CHECK(xnn_energy_stress_finish(XNN_F32, nullptr, 10, XNN_F32, virial, XNN_F32, virial,
                                 nullptr, 1.0, out, virial, nullptr) == XNN_EINVAL);
  CHECK(xnn_segment_reduce_f64(XNN_F32, nullptr, -1, 1, nullptr, 1, out, nullptr, 0,
                               nullptr) == XNN_EINVAL);
  CHECK(xnn_segment_reduce_f64(5, out, 10, 1, nullptr, 1, out, nullptr, 0, nullptr) ==
        XNN_EINVAL);
  CHECK(xnn_virial_finish(XNN_F32, nullptr, nullptr, -1, 1, virial, nullptr) == XNN_EINVAL);
  CHECK(xnn_stress_finish(XNN_F32, nullptr, XNN_F32, nullptr, nullptr, -1, 1.0, virial,
                          nullptr) == XNN_EINVAL);
  // a long error message stays within the thread's buffer
  CHECK(std::strlen(xnn_last_error()) < 4096);
}

int main() {
  CHECK(xnn_abi_version() == 2);
  plans();
  workspaces();
  argument_errors();
  if (failures == 0) std::printf("host ABI checks passed\n");
  return failures == 0 ? 0 : 1;
}
