/*
 * moe_index.c — plain-C restatement of the MoE routing index build
 * (TEST INFRASTRUCTURE ONLY; never linked into libmk).
 *
 * Follows, for one rank owning local experts [e0, e0+n_local) and a single
 * token source (node 0, dev 0):
 *   build_routing / padded_list     reference bench/dispatch_gemm_bench.py:127-166
 *   build_pull_indices              reference bench/dispatch_gemm_bench.py:169-188
 *   build_gather_indices            reference bench/dispatch_gemm_glu_combine_bench.py:222-293
 * It is written independently of libmk's C++ builder (counting sort per
 * expert instead of per-expert lists) so that the two cross-check.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int oracle_moe_sizes(const int32_t* ids, int32_t T, int32_t k, int32_t e0, int32_t n_local,
                     int32_t rb, int64_t* R, int64_t* R_pad) {
  int64_t* cnt = calloc((size_t)n_local, sizeof(int64_t));
  if (!cnt) return -1;
  for (int64_t i = 0; i < (int64_t)T * k; ++i) {
    int32_t e = ids[i] - e0;
    if (e >= 0 && e < n_local) cnt[e]++;
  }
  *R = 0;
  *R_pad = 0;
  for (int32_t e = 0; e < n_local; ++e) {
    *R += cnt[e];
    *R_pad += (cnt[e] + rb - 1) / rb * rb;
  }
  free(cnt);
  return 0;
}

/* Outputs (all caller-allocated): padded[n_local], pull[R_pad*3],
 * row_expert[R_pad], row_weight[R_pad], owner_offset[T+1], row_to_slot[R_pad],
 * row_to_owner[R_pad], slot_to_row[R]. */
int oracle_moe_build(const int32_t* ids, const float* gates, int32_t T, int32_t k, int32_t e0,
                     int32_t n_local, int32_t rb, int32_t* padded, int32_t* pull, int32_t* row_expert,
                     float* row_weight, int32_t* owner_offset, int32_t* row_to_slot,
                     int32_t* row_to_owner, int32_t* slot_to_row) {
  int64_t* cnt = calloc((size_t)n_local + 1, sizeof(int64_t));
  int64_t* start = calloc((size_t)n_local + 1, sizeof(int64_t));
  int32_t* fill = calloc((size_t)n_local + 1, sizeof(int32_t));
  int32_t* tcount = calloc((size_t)T + 1, sizeof(int32_t));
  int32_t* trun = calloc((size_t)T + 1, sizeof(int32_t));
  if (!cnt || !start || !fill || !tcount || !trun) return -1;
  for (int64_t i = 0; i < (int64_t)T * k; ++i) {
    int32_t e = ids[i] - e0;
    if (e >= 0 && e < n_local) cnt[e]++;
  }
  int64_t R_pad = 0;
  for (int32_t e = 0; e < n_local; ++e) {
    start[e] = R_pad;
    padded[e] = (int32_t)((cnt[e] + rb - 1) / rb * rb);
    R_pad += padded[e];
  }
  for (int64_t r = 0; r < R_pad; ++r) {
    pull[3 * r] = pull[3 * r + 1] = pull[3 * r + 2] = -1;
    row_weight[r] = 0.0f;
    row_to_slot[r] = 0;
    row_to_owner[r] = -1;
  }
  for (int32_t e = 0; e < n_local; ++e)
    for (int64_t i = 0; i < padded[e]; ++i) row_expert[start[e] + i] = e;
  /* token-major scan places (t, k) pairs in token order inside each expert */
  for (int32_t t = 0; t < T; ++t)
    for (int32_t j = 0; j < k; ++j) {
      int32_t e = ids[(int64_t)t * k + j] - e0;
      if (e < 0 || e >= n_local) continue;
      int64_t r = start[e] + fill[e]++;
      pull[3 * r] = 0;
      pull[3 * r + 1] = 0;
      pull[3 * r + 2] = t;
      row_weight[r] = gates[(int64_t)t * k + j];
      tcount[t]++;
    }
  owner_offset[0] = 0;
  for (int32_t t = 0; t < T; ++t) owner_offset[t + 1] = owner_offset[t] + tcount[t];
  for (int64_t r = 0; r < R_pad; ++r) {
    if (pull[3 * r] < 0) continue;
    int32_t t = pull[3 * r + 2];
    int32_t s = owner_offset[t] + trun[t]++;
    row_to_slot[r] = s;
    row_to_owner[r] = 0;
    slot_to_row[s] = (int32_t)r;
  }
  free(cnt);
  free(start);
  free(fill);
  free(tcount);
  free(trun);
  return 0;
}
