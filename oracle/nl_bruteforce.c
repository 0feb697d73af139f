/* Brute-force periodic neighbour list (test infrastructure, CPU oracle).
 *
 * Restates the edge-set definition of the reference's `get_neighborhood`
 * (tace/dataset/neighbour_list.py:195-298, matscipy "ijSd" at 240-248):
 *   all ordered (i, j, S) with |r_j - r_i + S . cell|^2 < cutoff^2,
 *   minus (i == j and S == 0)                      (286-292),
 *   S forced to 0 along non-periodic axes          (295).
 * Every pair is tested against every admissible image: for the pair's
 * fractional separation df, image k ranges over
 *   ceil(-df_k - rc/h_k) .. floor(-df_k + rc/h_k),  h_k = plane spacing,
 * so positions outside the cell are handled exactly.  float64 throughout.
 *
 * Output order: i ascending, then j ascending, then S lexicographic.
 * Two calls: pass out_* = NULL to count, then fill.
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>

static void inv3(const double *a, double *o) {
    double det = a[0] * (a[4] * a[8] - a[5] * a[7]) - a[1] * (a[3] * a[8] - a[5] * a[6]) +
                 a[2] * (a[3] * a[7] - a[4] * a[6]);
    o[0] = (a[4] * a[8] - a[5] * a[7]) / det;
    o[1] = (a[2] * a[7] - a[1] * a[8]) / det;
    o[2] = (a[1] * a[5] - a[2] * a[4]) / det;
    o[3] = (a[5] * a[6] - a[3] * a[8]) / det;
    o[4] = (a[0] * a[8] - a[2] * a[6]) / det;
    o[5] = (a[2] * a[3] - a[0] * a[5]) / det;
    o[6] = (a[3] * a[7] - a[4] * a[6]) / det;
    o[7] = (a[1] * a[6] - a[0] * a[7]) / det;
    o[8] = (a[0] * a[4] - a[1] * a[3]) / det;
}

int64_t nl_bruteforce(const double *pos, int64_t n, const double *cell, const int32_t *pbc,
                      double cutoff, int64_t *out_i, int64_t *out_j, int64_t *out_s) {
    double inv[9];
    inv3(cell, inv);
    /* plane spacing h_k = 1/|column k of inv| (row-vector lattice convention) */
    double reach[3];
    for (int k = 0; k < 3; ++k) {
        double c0 = inv[0 * 3 + k], c1 = inv[1 * 3 + k], c2 = inv[2 * 3 + k];
        reach[k] = pbc[k] ? cutoff * sqrt(c0 * c0 + c1 * c1 + c2 * c2) : 0.0;
    }
    const double rc2 = cutoff * cutoff;
    int64_t cnt = 0;
    for (int64_t i = 0; i < n; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            double d[3] = {pos[3 * j] - pos[3 * i], pos[3 * j + 1] - pos[3 * i + 1],
                           pos[3 * j + 2] - pos[3 * i + 2]};
            double f[3];
            for (int k = 0; k < 3; ++k) f[k] = d[0] * inv[k] + d[1] * inv[3 + k] + d[2] * inv[6 + k];
            int64_t lo[3], hi[3];
            for (int k = 0; k < 3; ++k) {
                if (pbc[k]) {
                    lo[k] = (int64_t)ceil(-f[k] - reach[k]) - 1;
                    hi[k] = (int64_t)floor(-f[k] + reach[k]) + 1;
                } else {
                    lo[k] = hi[k] = 0;
                }
            }
            for (int64_t a = lo[0]; a <= hi[0]; ++a)
                for (int64_t b = lo[1]; b <= hi[1]; ++b)
                    for (int64_t c = lo[2]; c <= hi[2]; ++c) {
                        if (i == j && a == 0 && b == 0 && c == 0) continue;
                        double v0 = d[0] + a * cell[0] + b * cell[3] + c * cell[6];
                        double v1 = d[1] + a * cell[1] + b * cell[4] + c * cell[7];
                        double v2 = d[2] + a * cell[2] + b * cell[5] + c * cell[8];
                        double r2 = v0 * v0 + v1 * v1 + v2 * v2;
                        if (r2 < rc2) {
                            if (out_i) {
                                out_i[cnt] = i;
                                out_j[cnt] = j;
                                out_s[3 * cnt] = a;
                                out_s[3 * cnt + 1] = b;
                                out_s[3 * cnt + 2] = c;
                            }
                            ++cnt;
                        }
                    }
        }
    }
    return cnt;
}
