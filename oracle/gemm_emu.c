/*
 * CPU emulation of the fp32 symmetric products of the coupled-Newton root
 * kernels -- TEST INFRASTRUCTURE ONLY (the oracle's product hook, used by
 * tests/golden/config4_emulated.py; nothing in the product links it).
 *
 * The reference computes each product with torch.matmul
 * (pytorch_opt/ops/reference.py:17-40); this restates the summation order
 * the library's fp32 MFMA core uses for those products (blocked
 * accumulation), so that the oracle's iteration can be run with the
 * kernel's product rounding:
 *   C(i,j) = sum over K tiles t of chain_t(i,j), added into the running sum
 *            in tile order (acc = acc + chain, one fp32 rounding each);
 *   chain_t = a fresh sequential fused multiply-add chain over the tile's
 *            16 k values, in the order the 16x16x4 MFMA feeds them: lane
 *            group g supplies k = 4g + ii in instruction ii, and each
 *            instruction applies its four k in lane-group order, so
 *            k = 0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15 (+16 t);
 *   symmetric products store the value computed for (min(i,j), max(i,j)) at
 *   both positions (upper tiles, mirrored).
 * Operands are row-major n x n with Q symmetric (the kernels read Q's rows
 * as its columns): C = P·Q. n must be a multiple of 16 here (the kernels
 * zero-pad K to a multiple of 128; the sizes emulated are multiples of 128,
 * so no pad terms enter the chains).
 *
 * Build: oracle/Makefile (gcc -O3 -mfma -fopenmp -ffp-contract=off); fmaf
 * is the exactly rounded fused operation and nothing else is contracted.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

static const int kOrder[16] = {0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15};

/* C[i][j] for j >= i (mirrored into C[j][i]); Qt = Q transposed (so the
 * inner loop over j reads contiguous memory). blocked = 0 instead runs one
 * sequential chain over k = 0 .. n-1 (a plain FMA loop: the planted
 * difference the tests use to show the emulation is order-sensitive).
 * Returns 0, or -1 if n is not a multiple of 16 or memory runs out. */
int emu_sym_product_f32(const float* P, const float* Q, float* C, int n, int blocked) {
  if (n <= 0 || n % 16 != 0) return -1;
  float* Qt = (float*)malloc(sizeof(float) * (size_t)n * n);
  if (!Qt) return -1;
  for (int k = 0; k < n; ++k)
    for (int j = 0; j < n; ++j) Qt[(size_t)k * n + j] = Q[(size_t)j * n + k];
  int fail = 0;
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * n);
    float* t = (float*)malloc(sizeof(float) * n);
    if (!acc || !t) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(dynamic, 4)
      for (int i = 0; i < n; ++i) {
        const int j0 = i;  /* the upper part of row i */
        const int w = n - j0;
        memset(acc + j0, 0, sizeof(float) * w);
        if (!blocked) {
          for (int k = 0; k < n; ++k) {
            const float p = P[(size_t)i * n + k];
            const float* qrow = Qt + (size_t)k * n;
            for (int j = j0; j < n; ++j) acc[j] = fmaf(p, qrow[j], acc[j]);
          }
        }
        for (int kt = 0; blocked && kt < n; kt += 16) {
          memset(t + j0, 0, sizeof(float) * w);
          for (int q = 0; q < 16; ++q) {
            const int k = kt + kOrder[q];
            const float p = P[(size_t)i * n + k];
            const float* qrow = Qt + (size_t)k * n;
            for (int j = j0; j < n; ++j) t[j] = fmaf(p, qrow[j], t[j]);
          }
          for (int j = j0; j < n; ++j) acc[j] = acc[j] + t[j];
        }
        for (int j = j0; j < n; ++j) {
          C[(size_t)i * n + j] = acc[j];
          C[(size_t)j * n + i] = acc[j];
        }
      }
    }
    free(acc);
    free(t);
  }
  free(Qt);
  return fail ? -1 : 0;
}
