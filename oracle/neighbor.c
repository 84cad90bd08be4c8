/*
 * TEST INFRASTRUCTURE ONLY -- the oracle of the radius graph, never the product.
 *
 * A CPU restatement of the reference's brute-force neighbor list,
 * build_neighbor_list (src/xnn/common/data/neighborlist.py:462-506), for one
 * structure, in the positions' own precision (float or double):
 *   1. wrap along periodic axes: frac = pos @ inv(cell), o = floor(frac) (zeroed on
 *      non-periodic axes), w = pos - o @ cell                       (lines 472-475)
 *   2. image shifts S in itertools.product order over [-r, r]^3,
 *      shift vectors S @ cell                                        (lines 476-481)
 *   3. rij = (w_j - w_i) + S @ cell, dist = |rij|, keep dist < cutoff (lines 483-486)
 *   4. drop i == j in the zero image unless self_interaction         (lines 487-490)
 *   5. edge (src = j, dst = i), shift = -S + o_j - o_i, in the order of
 *      torch.nonzero over (S, i, j)                                  (lines 492-505)
 * The norm is accumulated in double and rounded to the geometry type before the
 * comparison (a CPU float reduction accumulates in double). `near` counts pairs whose
 * double-precision distance lies within `margin` of the cutoff: where it is zero, no
 * rounding of the distance can move a pair across the cutoff.
 *
 * Count pass: oracle_nl_count_<t>(...) fills counts[S*N] (edges of image s and
 * receiver i) and returns their total; the caller turns them into offsets and runs
 * oracle_nl_fill_<t>(...). Parallel over receivers with OpenMP; the output order
 * does not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_NL(T, SUFFIX)                                                                 \
  static void wrap_##SUFFIX(const T* pos, int64_t n, const T* cell, const T* inv,            \
                            const int32_t* pbc, T* w, int64_t* off) {                       \
    for (int64_t i = 0; i < n; ++i) {                                                        \
      int64_t o[3] = {0, 0, 0};                                                              \
      if (cell) {                                                                            \
        for (int a = 0; a < 3; ++a) {                                                        \
          T f = pos[3 * i] * inv[a] + pos[3 * i + 1] * inv[3 + a] + pos[3 * i + 2] * inv[6 + a]; \
          o[a] = pbc[a] ? (int64_t)floor((double)f) : 0;                                     \
        }                                                                                    \
      }                                                                                      \
      for (int a = 0; a < 3; ++a) {                                                          \
        T sub = 0;                                                                           \
        if (cell) sub = (T)o[0] * cell[a] + (T)o[1] * cell[3 + a] + (T)o[2] * cell[6 + a];   \
        w[3 * i + a] = (o[0] | o[1] | o[2]) ? pos[3 * i + a] - sub : pos[3 * i + a];         \
        off[3 * i + a] = o[a];                                                               \
      }                                                                                      \
    }                                                                                        \
  }                                                                                          \
  static int64_t n_images_##SUFFIX(const int32_t* reps) {                                    \
    return (int64_t)(2 * reps[0] + 1) * (2 * reps[1] + 1) * (2 * reps[2] + 1);              \
  }                                                                                          \
  static void image_##SUFFIX(const int32_t* reps, int64_t s, int64_t* S) {                   \
    const int64_t ny = 2 * reps[1] + 1, nz = 2 * reps[2] + 1;                                \
    S[0] = s / (ny * nz) - reps[0];                                                          \
    S[1] = (s / nz) % ny - reps[1];                                                          \
    S[2] = s % nz - reps[2];                                                                 \
  }                                                                                          \
  static int test_##SUFFIX(const T* w, int64_t i, int64_t j, const T* sv, T cutoff,          \
                           double margin, int64_t* near) {                                  \
    const T dx = (w[3 * j] - w[3 * i]) + sv[0];                                              \
    const T dy = (w[3 * j + 1] - w[3 * i + 1]) + sv[1];                                      \
    const T dz = (w[3 * j + 2] - w[3 * i + 2]) + sv[2];                                      \
    const double d2 = (double)dx * dx + (double)dy * dy + (double)dz * dz;                  \
    const double d = sqrt(d2);                                                               \
    if (near && fabs(d - (double)cutoff) < margin) ++*near;                                  \
    return (T)d < cutoff;                                                                    \
  }                                                                                          \
  int64_t oracle_nl_count_##SUFFIX(const T* pos, int64_t n, const T* cell, const T* inv,    \
                                   const int32_t* pbc, const int32_t* reps, T cutoff,        \
                                   int self_interaction, double margin, int64_t* counts,     \
                                   int64_t* near_out) {                                      \
    T* w = (T*)malloc(sizeof(T) * 3 * (n > 0 ? n : 1));                                     \
    int64_t* off = (int64_t*)malloc(sizeof(int64_t) * 3 * (n > 0 ? n : 1));                  \
    wrap_##SUFFIX(pos, n, cell, inv, pbc, w, off);                                           \
    const int64_t ns = n_images_##SUFFIX(reps);                                              \
    int64_t total = 0, near = 0;                                                             \
    for (int64_t s = 0; s < ns; ++s) {                                                       \
      int64_t S[3];                                                                          \
      image_##SUFFIX(reps, s, S);                                                            \
      T sv[3] = {0, 0, 0};                                                                   \
      if (cell)                                                                              \
        for (int a = 0; a < 3; ++a)                                                          \
          sv[a] = (T)S[0] * cell[a] + (T)S[1] * cell[3 + a] + (T)S[2] * cell[6 + a];         \
      const int zero = S[0] == 0 && S[1] == 0 && S[2] == 0;                                  \
      _Pragma("omp parallel for schedule(static) reduction(+ : total, near)")                \
      for (int64_t i = 0; i < n; ++i) {                                                      \
        int64_t c = 0;                                                                       \
        for (int64_t j = 0; j < n; ++j) {                                                    \
          if (test_##SUFFIX(w, i, j, sv, cutoff, margin, &near)) {                           \
            if (!self_interaction && zero && i == j) continue;                               \
            ++c;                                                                             \
          }                                                                                  \
        }                                                                                    \
        counts[s * n + i] = c;                                                               \
        total += c;                                                                          \
      }                                                                                      \
    }                                                                                        \
    free(w);                                                                                 \
    free(off);                                                                               \
    if (near_out) *near_out = near;                                                          \
    return total;                                                                            \
  }                                                                                          \
  void oracle_nl_fill_##SUFFIX(const T* pos, int64_t n, const T* cell, const T* inv,        \
                               const int32_t* pbc, const int32_t* reps, T cutoff,            \
                               int self_interaction, const int64_t* offsets, int64_t n_edges, \
                               int64_t* edge_index, int64_t* shifts) {                       \
    T* w = (T*)malloc(sizeof(T) * 3 * (n > 0 ? n : 1));                                     \
    int64_t* off = (int64_t*)malloc(sizeof(int64_t) * 3 * (n > 0 ? n : 1));                  \
    wrap_##SUFFIX(pos, n, cell, inv, pbc, w, off);                                           \
    const int64_t ns = n_images_##SUFFIX(reps);                                              \
    for (int64_t s = 0; s < ns; ++s) {                                                       \
      int64_t S[3];                                                                          \
      image_##SUFFIX(reps, s, S);                                                            \
      T sv[3] = {0, 0, 0};                                                                   \
      if (cell)                                                                              \
        for (int a = 0; a < 3; ++a)                                                          \
          sv[a] = (T)S[0] * cell[a] + (T)S[1] * cell[3 + a] + (T)S[2] * cell[6 + a];         \
      const int zero = S[0] == 0 && S[1] == 0 && S[2] == 0;                                  \
      _Pragma("omp parallel for schedule(static)")                                           \
      for (int64_t i = 0; i < n; ++i) {                                                      \
        int64_t e = offsets[s * n + i];                                                      \
        for (int64_t j = 0; j < n; ++j) {                                                    \
          if (!test_##SUFFIX(w, i, j, sv, cutoff, 0.0, NULL)) continue;                      \
          if (!self_interaction && zero && i == j) continue;                                 \
          edge_index[e] = j;                                                                 \
          edge_index[n_edges + e] = i;                                                       \
          for (int a = 0; a < 3; ++a) shifts[3 * e + a] = -S[a] + off[3 * j + a] - off[3 * i + a]; \
          ++e;                                                                               \
        }                                                                                    \
      }                                                                                      \
    }                                                                                        \
    free(w);                                                                                 \
    free(off);                                                                               \
  }

ORACLE_NL(float, f32)
ORACLE_NL(double, f64)
