/*
 * C-language check of the mlxvs C ABI (include/mlxvs/mlxvs_c.h), in the
 * style of the reference's tests/test_c_api.c:247-258: the header compiles as
 * C, the library links, and invalid arguments give MLXVS_ERROR_INVALID_ARGUMENT
 * with a non-empty mlxvs_last_error() before any GPU work.  With
 * MLXVS_EXPECT_GPU=0 (no GPU), a valid call must fail with
 * MLXVS_ERROR_INTERNAL: there is no CPU fallback.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mlxvs/mlxvs_c.h"

static int failures = 0;

static void check(int ok, const char* what) {
  if (!ok) {
    ++failures;
    printf("FAIL %s\n", what);
  }
}

int main(void) {
  float rows[8] = {0};
  int32_t ids[16];
  float dist[16];
  uint8_t codes[8] = {0};
  printf("mlxvs %s, C API %d\n", mlxvs_version(), MLXVS_C_API_VERSION);
  check(strcmp(mlxvs_version(), "0.16.1") == 0, "version");
  check(MLXVS_INNER_PRODUCT == 0 && MLXVS_L2 == 1 && MLXVS_COSINE == 2, "metric values");
  check(MLXVS_OK == 0 && MLXVS_ERROR_INVALID_ARGUMENT == 1 && MLXVS_ERROR_IO == 2 &&
            MLXVS_ERROR_INTERNAL == 3, "status values");

  int st = mlxvs_brute_force_knn(rows, 2, rows, 1, 4, 1, MLXVS_L2, NULL, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT && strlen(mlxvs_last_error()) > 0, "NULL ids");
  st = mlxvs_brute_force_knn(rows, 2, rows, 1, 4, 1, (mlxvs_metric)7, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT && strlen(mlxvs_last_error()) > 0, "bad metric");
  st = mlxvs_brute_force_knn(rows, 2, rows, 1, 4, 300, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "k = 300");
  st = mlxvs_brute_force_knn(rows, 2, rows, 1, 4, 0, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "k = 0");
  st = mlxvs_brute_force_knn(NULL, 2, rows, 1, 4, 1, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "NULL base");
  st = mlxvs_brute_force_knn(rows, -1, rows, 1, 4, 1, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "n < 0");
  st = mlxvs_brute_force_knn(rows, 2, rows, 1, 0, 1, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "d < 1");
  st = mlxvs_hamming_knn(codes, 2, codes, 1, 4, 0, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "hamming k = 0");
  st = mlxvs_hamming_knn(codes, 2, codes, 1, 4, 257, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "hamming k = 257");
  st = mlxvs_knn_self_graph(rows, 1, 4, 0, 3, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "self graph n < 2");
  st = mlxvs_knn_self_graph(rows, 2, 4, 0, 256, MLXVS_L2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "self graph k = 256");

  float scores[6] = {0};
  st = mlxvs_topk_merge(scores, 2, 3, NULL, NULL, 0, 1, 0, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT &&
            strstr(mlxvs_last_error(), "[mlxvs::topk_merge] k must be in [1, 256]") != NULL,
        "topk_merge k = 0");
  st = mlxvs_topk_merge(scores, 2, 3, NULL, NULL, 0, 0, 2, ids, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "topk_merge running lists NULL unless first");
  st = mlxvs_topk_merge(scores, 2, 3, NULL, NULL, 0, 1, 2, NULL, dist);
  check(st == MLXVS_ERROR_INVALID_ARGUMENT, "topk_merge NULL out_ids");
  st = mlxvs_topk_merge(scores, 0, 3, NULL, NULL, 0, 1, 2, ids, dist);
  check(st == MLXVS_OK, "topk_merge with no rows does nothing");

  st = mlxvs_profile(0);
  check(st == MLXVS_OK && strlen(mlxvs_last_error()) == 0, "success clears the error");

  const char* expect_gpu = getenv("MLXVS_EXPECT_GPU");
  if (expect_gpu && strcmp(expect_gpu, "0") == 0) {
    st = mlxvs_brute_force_knn(rows, 2, rows, 1, 4, 1, MLXVS_L2, ids, dist);
    check(st == MLXVS_ERROR_INTERNAL && strlen(mlxvs_last_error()) > 0,
          "no GPU: the call fails (no CPU fallback)");
  }
  printf(failures == 0 ? "all tests passed\n" : "%d FAILED\n", failures);
  return failures == 0 ? 0 : 1;
}
