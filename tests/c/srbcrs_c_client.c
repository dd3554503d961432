/* A plain C99 client of the C ABI (include/srbcrs.h), test infrastructure:
 * builds a seeded random CSR on the host, converts it (host CSR, then the
 * device converter from HBM), runs the SpMM with default and tuned launch
 * settings and the nonzero sweep, and checks C against a double-precision
 * loop on the host with the fp32 gate |C - C64| <= 1e-4 * (|A||B|).
 * Prints "C-ABI OK" and returns 0 on success. */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "srbcrs.h"

#define CHECK(call)                                                              \
  do {                                                                           \
    int rc_ = (call);                                                            \
    if (rc_ != SRBCRS_OK) {                                                      \
      fprintf(stderr, "%s failed (%d): %s\n", #call, rc_, srbcrs_last_error());  \
      return 1;                                                                  \
    }                                                                            \
  } while (0)
#define HIPCHECK(call)                                                           \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));          \
      return 1;                                                                  \
    }                                                                            \
  } while (0)

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint32_t next_u32(void) {
  state ^= state << 13;
  state ^= state >> 7;
  state ^= state << 17;
  return (uint32_t)(state >> 11);
}

static int check(const float *C, const int32_t *rp, const int32_t *ci, const float *v, const float *B,
                 int M, int N) {
  for (int r = 0; r < M; ++r)
    for (int j = 0; j < N; ++j) {
      double s = 0.0, a = 0.0;
      for (int e = rp[r]; e < rp[r + 1]; ++e) {
        s += (double)v[e] * B[(size_t)ci[e] * N + j];
        a += fabs((double)v[e] * B[(size_t)ci[e] * N + j]);
      }
      if (fabs((double)C[(size_t)r * N + j] - s) > 1e-4 * a + 1e-30) {
        fprintf(stderr, "mismatch at (%d, %d): %g vs %g\n", r, j, C[(size_t)r * N + j], s);
        return 1;
      }
    }
  return 0;
}

int main(void) {
  const int M = 1000, K = 1200, N = 128;
  int32_t *rp = malloc(sizeof(int32_t) * (M + 1));
  int32_t *ci = malloc(sizeof(int32_t) * M * 24);
  float *v = malloc(sizeof(float) * M * 24);
  rp[0] = 0;
  for (int r = 0; r < M; ++r) {   /* distinct, sorted columns per row: no duplicates */
    int n = (int)(next_u32() % 24), c = (int)(next_u32() % 40);
    for (int k = 0; k < n && c < K; ++k) {
      ci[rp[r] + k] = c;
      v[rp[r] + k] = (float)((int)(next_u32() % 2001) - 1000) / 1000.0f;
      c += 1 + (int)(next_u32() % 90);
      rp[r + 1] = rp[r] + k + 1;
    }
    if (n == 0 || rp[r + 1] < rp[r]) rp[r + 1] = rp[r];
  }
  const int64_t nnz = rp[M];
  float *B = malloc(sizeof(float) * K * N), *C = malloc(sizeof(float) * M * N);
  for (int i = 0; i < K * N; ++i) B[i] = (float)((int)(next_u32() % 2001) - 1000) / 1000.0f;

  float *dB, *dC;
  int32_t *drp, *dci;
  float *dv;
  HIPCHECK(hipMalloc((void **)&dB, sizeof(float) * K * N));
  HIPCHECK(hipMalloc((void **)&dC, sizeof(float) * M * N));
  HIPCHECK(hipMalloc((void **)&drp, sizeof(int32_t) * (M + 1)));
  HIPCHECK(hipMalloc((void **)&dci, sizeof(int32_t) * (nnz ? nnz : 1)));
  HIPCHECK(hipMalloc((void **)&dv, sizeof(float) * (nnz ? nnz : 1)));
  HIPCHECK(hipMemcpy(dB, B, sizeof(float) * K * N, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(drp, rp, sizeof(int32_t) * (M + 1), hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(dci, ci, sizeof(int32_t) * nnz, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(dv, v, sizeof(float) * nnz, hipMemcpyHostToDevice));

  for (int path = 0; path < 2; ++path) {
    srbcrs_plan *plan = NULL;
    if (path == 0)
      CHECK(srbcrs_plan_create(rp, ci, v, M, nnz, 16, 8, 0, NULL, &plan));      /* host CSR */
    else
      CHECK(srbcrs_plan_create(drp, dci, dv, M, nnz, 16, 8, 1, NULL, &plan));   /* device CSR */
    srbcrs_plan_desc d;
    CHECK(srbcrs_plan_get(plan, &d));
    if (d.row_windows != (M + 15) / 16 || d.nnz != nnz) {
      fprintf(stderr, "bad plan description\n");
      return 1;
    }
    CHECK(srbcrs_plan_set_schedule(plan, "auto", 0));
    CHECK(srbcrs_run(plan, dB, K, N, N, dC, N, M, NULL));
    HIPCHECK(hipMemcpy(C, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost));
    if (check(C, rp, ci, v, B, M, N)) return 1;
    srbcrs_run_opts best;
    CHECK(srbcrs_plan_tune(plan, dB, K, N, N, dC, N, M, 2, &best, NULL));
    HIPCHECK(hipMemset(dC, 0, sizeof(float) * M * N));
    CHECK(srbcrs_run(plan, dB, K, N, N, dC, N, M, NULL));   /* uses the tuned setting */
    HIPCHECK(hipMemcpy(C, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost));
    if (check(C, rp, ci, v, B, M, N)) return 1;
    /* the nonzero sweep (grid order 5, row schedule), then the tuner with it admitted */
    CHECK(srbcrs_plan_set_schedule(plan, "row", 0));
    srbcrs_run_opts sweep = {0};
    sweep.grid_order = SRBCRS_GRID_NZSWEEP;
    HIPCHECK(hipMemset(dC, 0, sizeof(float) * M * N));
    CHECK(srbcrs_run_ex(plan, dB, K, N, N, dC, N, M, &sweep, NULL));
    HIPCHECK(hipMemcpy(C, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost));
    if (check(C, rp, ci, v, B, M, N)) return 1;
    CHECK(srbcrs_plan_tune_ex(plan, dB, K, N, N, dC, N, M, 2, SRBCRS_TUNE_NONZERO_SWEEP, &best, NULL));
    HIPCHECK(hipMemset(dC, 0, sizeof(float) * M * N));
    CHECK(srbcrs_run(plan, dB, K, N, N, dC, N, M, NULL));
    HIPCHECK(hipMemcpy(C, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost));
    if (check(C, rp, ci, v, B, M, N)) return 1;
    /* the relu epilogue on the tuned setting: relu of the plain output, bit for bit */
    {
      srbcrs_run_opts relu = {0};
      relu.epilogue = SRBCRS_EPILOGUE_RELU;
      float* R = (float*)malloc(sizeof(float) * M * N);
      HIPCHECK(hipMemset(dC, 0, sizeof(float) * M * N));
      CHECK(srbcrs_run_ex(plan, dB, K, N, N, dC, N, M, &relu, NULL));
      HIPCHECK(hipMemcpy(R, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost));
      for (size_t i = 0; i < (size_t)M * N; ++i)
        if (R[i] != (C[i] < 0.f ? 0.f : C[i])) {
          fprintf(stderr, "relu epilogue mismatch at %zu: %g vs %g\n", i, R[i], C[i]);
          return 1;
        }
      free(R);
    }
    /* an error path: N not a multiple of 16 */
    if (srbcrs_run(plan, dB, K, 24, N, dC, N, M, NULL) != SRBCRS_EINVAL) {
      fprintf(stderr, "expected SRBCRS_EINVAL\n");
      return 1;
    }
    srbcrs_plan_destroy(plan);
  }
  hipFree(dB); hipFree(dC); hipFree(drp); hipFree(dci); hipFree(dv);
  free(rp); free(ci); free(v); free(B); free(C);
  printf("C-ABI OK (%s)\n", srbcrs_version());
  return 0;
}
