// mk_internal.h — kernel parameter blocks and launchers shared between the
// HIP translation units of libmk (not part of the C-ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mk {

enum Epilogue : int { kEpiStore = 0, kEpiSwiGLU = 1, kEpiReduce = 2 };
enum PermMode : int { kPermNone = 0, kPermArrival = 1, kPermOwnedSpread = 2, kPermPeerArrival = 3 };
constexpr int kMaxTilesM = 512;
constexpr int kMaxSplitListTiles = 4096;  // K-split with a permuted tile order: at most this many tiles
constexpr int kMaxRounds = 64;   // cooperative staging between rounds: at most this many rounds
constexpr int kPieces = 16;  // cooperative staging: pieces per 128-row block

struct GemmKParams {
  // operands
  const uint16_t* A;
  const uint16_t* B;
  uint16_t* C;
  int64_t lda, ldb, ldc;
  int64_t b_expert_stride;  // elements between experts' B matrices
  int M, N, K;
  int tiles_m, tiles_n;
  int group_m;
  // 128-row grouped GEMMs with rb_expert: walk each expert's run of row
  // tiles column by column (one expert's tiles consecutive) instead of the
  // grouped order
  int expert_order;
  // grid roles
  int n_prod, n_cons;
  int xcd_remap;
  int waves;                // 4 (one wave per SIMD) or 8 (two per SIMD)
  // grouped GEMM: expert of each BM row tile (nullptr = dense)
  const int* rb_expert;
  const int* expert_rows;   // padded rows per expert (used when rb_expert is null)
  const int* rb_rows;       // real rows per 128-row tile (null: every row is real)
  // fused dispatch: A is the token buffer [gather_rows, K], row r of the
  // GEMM reads the token the pull table names (null: A rows are the rows)
  const int* gather_pull;
  int64_t gather_rows;
  int gather_tps, gather_devs;
  int n_experts;
  // SwiGLU: width I of the gate half of B's columns
  int swiglu_I;
  // consumer A-row gate (AllGather side)
  const uint32_t* a_flags;
  const int* a_stage_order;
  int perm_mode;
  // reduce epilogue (ReduceScatter side)
  int rs_own_row0, rs_own_rows, rs_npeers;
  const uint16_t* rs_recv;
  uint16_t* rs_out;
  const uint32_t* rs_flags;
  uint32_t* ar_done;        // all-reduce: per output tile, epoch once its reduced bytes are visible
  // producer staging: block b (128 rows of st_cols) copied st_src -> st_dst
  const uint16_t* st_src;
  uint16_t* st_dst;
  int st_cols, st_nblocks;
  // Blocks at index >= st_split_at (when st_src2 is set) form a second
  // staging set: block st_split_at + b copies st_src2 block b to st_dst2
  // block b, or b + st_dst2_skip from block st_dst2_skip_at on (the
  // all-gather half of a two-shot all-reduce: the other slices' reduced
  // rows into C_final, around this rank's own slice).
  const uint16_t* st_src2;
  uint16_t* st_dst2;
  int st_split_at, st_dst2_skip_at, st_dst2_skip;
  int st_present;           // stage positions < st_present hold blocks already in st_dst: published, not copied
  const int* st_order;
  uint32_t* st_flags;
  uint32_t* st_counters;    // cooperative staging: pieces completed per block (mod kPieces)
  int st_coop;              // 1: even share, 2: alternating halves, 3: claimed (co-resident staging kernel)
  // st_coop 3: [0] the next unclaimed piece, shared with the staging kernel;
  // [1] claimers checked out; the last of st_claimers compute workgroups +
  // st_stage_waves staging waves to check out zeroes both
  uint32_t* st_claim;
  int st_claimers, st_stage_waves;
  int st_batch;             // pieces per release after the first (1..8)
  // K-split of the tail round: tiles >= sk_full are split sk_split ways along
  // K (sk_split <= 1: no split); partials go through sk_ws with sk_flags
  float* sk_ws;
  uint32_t* sk_flags;
  int sk_full, sk_split;
  // Device row count (128-row grouped GEMMs launched at a row capacity
  // before the routed row count is known on the host): *rows_dev rows are
  // real, tiles past them are not walked, and with sk_dev the tail round's
  // K-split is planned on the device by the host's rule (sk_ws / sk_flags
  // then hold n_cons partial tiles).
  const int64_t* rows_dev;
  int sk_dev;
  int spread_dev;           // with rows_dev: spread an unsplittable tail over fewer consumers (host rule)
  // flag protocol: the epoch is *epoch_ptr when that is set (read once per
  // use at run time, written by an earlier launch), else `epoch`
  const uint32_t* epoch_ptr;
  uint32_t epoch;
  uint32_t spin_limit;
  uint32_t* err;
};

hipError_t launch_gemm(const GemmKParams& p, int bm, int epi, hipStream_t stream, int bn = 256);
// Co-resident staging: the one-wave staging kernel (waves_per_cu per CU)
// followed by a register-capped 256 x 256 GEMM that may start while the
// staging kernel runs; both claim pieces through p.st_claim.
hipError_t launch_gemm_costaged(const GemmKParams& p, int epi, int n_stage_waves, hipStream_t stream);
hipError_t launch_epoch_advance(uint32_t* epoch_ptr, hipStream_t stream);

struct PermuteKParams {
  const uint16_t* tokens;
  const int* pull;
  uint16_t* post;
  int64_t R_pad, H, n_src_rows;
  int tokens_per_src, devs_per_node;
  const int64_t* rows_dev;  // device row count (rows at or past it are skipped), or null
};
hipError_t launch_permute(const PermuteKParams& p, hipStream_t stream);

struct CombineKParams {
  const uint16_t* y_expert;
  const float* row_weight;
  const int* owner_offset;
  const int* slot_to_row;
  void* y_out;
  int64_t num_tokens, H;
  int out_dtype;
};
hipError_t launch_combine(const CombineKParams& p, hipStream_t stream);
hipError_t launch_tile_rows(const int* pull, int64_t R_pad, int* rb_rows, hipStream_t stream);
int64_t index_workspace_bytes(int T, int topk, int n_local);
hipError_t launch_mfma_ceiling(int64_t iters, int n_wg, uint32_t seed, float* sink, uint64_t* clocks,
                               hipStream_t stream);
int probe_threads();
hipError_t launch_invert_slots(const int* row_to_slot, const int* row_to_owner, int64_t R_pad, int owner,
                               int64_t slot_capacity, int* slot_to_row, uint32_t* err, hipStream_t stream);

}  // namespace mk
