/*
 * mk.h — C-ABI of libmk, the MI355X (gfx950) compute core behind mKernel's
 * fused operators at one GPU's share of the work.
 *
 * Plain pointers and sizes only; no torch types.  Every device pointer is a
 * HIP device address; `stream` is a hipStream_t passed as void* (NULL = the
 * default stream).  All tensors are caller-owned and row-major.  bf16 buffers
 * are raw 16-bit storage (IEEE bfloat16).
 *
 * Return codes: 0 = ok, negative = argument/shape error (MK_E*), positive =
 * a hipError_t from a launch.  mk_last_error_string() describes the last
 * non-zero return on the calling thread.
 *
 * Each entry point names the reference interface it replaces (file:line in
 * uccl-project/mKernel).
 */
#ifndef MK_H_
#define MK_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MK_OK 0
#define MK_EINVAL (-1)   /* null pointer / bad enum */
#define MK_ESHAPE (-2)   /* shape not supported by the tiling */
#define MK_EDEVICE (-3)  /* no usable device / wrong architecture */
#define MK_ETIMEOUT (-4) /* a bounded flag wait expired (error word set) */

#define MK_ROW_BLOCK 128 /* flag / expert-padding granularity (rows) */

/* ------------------------------------------------------------------------ */
/* Plain persistent bf16 GEMM: C[M,N] = A[M,K] @ B[K,N], fp32 accumulate,
 * bf16 (round-to-nearest-even) output.
 * Replaces the compute role shared by ag_gemm / gemm_rs
 * (reference src/gemm_rs.cu:36-114 compute_tile_impl,
 *  src/ag_gemm.cu:265-461 fused_comp_sm).
 * Requires M % 128 == 0, N % 256 == 0, K % 32 == 0, ld* >= row width and
 * ld* % 8 == 0. */
typedef struct mk_gemm_args {
  const void* A;  /* bf16 [M, lda] */
  const void* B;  /* bf16 [K, ldb] */
  void* C;        /* bf16 [M, ldc] */
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int32_t num_cus; /* persistent grid size; 0 = every CU of the device; at most the CU count */
  int32_t tile_m;  /* 0 = auto (256 unless 128-row tiles fit in one round
                      of the grid), else 128 or 256 */
  int32_t waves;   /* waves per workgroup: 0 = auto, 4 (one per SIMD) or 8 (two per SIMD) */
  void* split_ws;          /* optional K-split workspace (see mk_query_workspace_bytes);
                              zero-filled before its first use, left zeroed by every
                              launch; NULL = no K-split of the tail round */
  int64_t split_ws_bytes;
} mk_gemm_args;
int mk_gemm(const mk_gemm_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Flag-gated AllGather+GEMM consumer with an in-GPU producer role.
 * C[M,N] = A_full[M,K] @ B[K,N].  A_full is assembled from `world` row
 * shards: `num_producers` producer workgroups copy 128-row tiles of
 * A_shards into A_full in the order `stage_order` and release-store
 * flags[tile] = epoch after each tile; compute workgroups acquire-poll the
 * flags of the rows they are about to read (s_sleep between polls).
 * Replaces ag_gemm_multinode::entrypoint
 * (reference include/operators/ag_gemm/ag_gemm.cuh:362-509) with the
 * intra_comm_sm gather role (src/ag_gemm.cu:31-215) and the per-chunk flag
 * wait of fused_comp_sm (src/ag_gemm.cu:374-377).
 *   gated == 0             : plain GEMM on A_full, no flags read (baseline)
 *   gated, producers == 0  : flags are published by someone else
 *   gated, producers  > 0  : that many producer workgroups run inside the
 *                            launch beside the compute workgroups
 *   gated, producers == -1 : cooperative staging — the compute workgroups
 *                            copy 128 KB pieces (in stage order) between
 *                            their tile rounds, counting pieces per tile in
 *                            stage_counters; the workgroup that completes a
 *                            tile publishes its flag.  Before round 0 every
 *                            workgroup copies what round 0 waits for; after
 *                            that the two halves of the grid (XCDs 0-3 and
 *                            4-7) take turns: one copies ahead for the next
 *                            round while the other computes
 *   gated, producers == -2 : cooperative staging with every workgroup
 *                            copying an even share before every round
 *   gated, producers <= -3 : wave-specialised producer: a staging kernel of
 *                            (-2 - producers) one-wave workgroups per
 *                            compute workgroup (1..4) runs beside a GEMM
 *                            capped at 224 VGPRs (room for one 64-VGPR
 *                            staging wave per SIMD) on a library side
 *                            stream, forked from and joined back into
 *                            `stream`; pieces are claimed in stage order
 *                            from a word in split_ws (required), the
 *                            compute workgroups claiming what a round
 *                            still lacks.  Under graph capture the call
 *                            stages cooperatively (-1) instead.  Needs
 *                            stage_counters. */
typedef struct mk_ag_gemm_args {
  const void* A_shards;  /* bf16 [M, K]: shards stacked in rank order (source) */
  void* A_full;          /* bf16 [M, K]: gathered A (destination / GEMM input) */
  const void* B;         /* bf16 [K, N] */
  void* C;               /* bf16 [M, N] */
  int64_t M, N, K;
  uint32_t* flags;              /* [M/128] epoch-stamped ready flags */
  const int32_t* stage_order;   /* [M/128] device; NULL = ascending */
  uint32_t epoch;               /* value a ready flag must hold (never 0) */
  int32_t gated;
  int32_t num_producers;
  int32_t num_cus;              /* total workgroups (producers + compute); 0 = all CUs; never more
                                   than the device's CUs (every workgroup must be resident) */
  uint32_t spin_limit;          /* polls before a wait gives up; 0 = unbounded */
  uint32_t* error_word;         /* optional device word, bit0 set on timeout */
  uint32_t* stage_counters;     /* [M/128] piece counters for producers == -1; zero once, never reset */
  void* split_ws;          /* optional K-split workspace (see mk_query_workspace_bytes);
                              zero-filled before its first use, left zeroed by every
                              launch; NULL = no K-split of the tail round */
  int64_t split_ws_bytes;
  /* Optional device word holding the epoch: when set, the launch reads the
   * epoch from it (never 0) instead of `epoch`, so a HIP graph that records
   * mk_epoch_advance and this launch gates every replay on a new epoch with
   * no host work.  NULL = use `epoch`. */
  const uint32_t* epoch_ptr;
  /* Number of leading stage_order positions whose 128-row blocks are
   * already in A_full (this rank's own shard, written there by the caller
   * as the reference bench does, bench/ag_gemm_bench.py:364-372): the
   * staging publishes their flags without copying them, and A_shards is
   * not read for them.  0 = every block is copied.  Needs stage_order when
   * non-zero. */
  int32_t n_present;
} mk_ag_gemm_args;
int mk_ag_gemm(const mk_ag_gemm_args* args, void* stream);

/* mk_ag_gemm without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * K-split workspace and the cooperative-staging piece counters come from a
 * static device array of mk_ag_gemm_noalloc_scratch_bytes() bytes (about
 * 32 MB, one copy per GPU, held until the process ends); split_ws,
 * split_ws_bytes and stage_counters must be NULL / 0.  Limits: M/128 <=
 * 16384 row blocks (larger M returns MK_ESHAPE); a tail round whose K-split
 * would need more than 128 partial tiles runs unsplit; num_producers <= -3
 * (the co-resident staging kernel, whose side stream and events the library
 * creates on first use) stages cooperatively (-1) instead.  Each call checks
 * every argument, then clears the counters, split flags and claim words it
 * uses on `stream` (a small kernel), then launches mk_ag_gemm's kernels.  Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (different streams)
 * race and must not be issued. */
int mk_ag_gemm_noalloc(const mk_ag_gemm_args* args, void* stream);
int64_t mk_ag_gemm_noalloc_scratch_bytes(void);

/* ------------------------------------------------------------------------ */
/* GEMM + reduce-scatter epilogue at one rank's share.
 * P = A[M,K] @ B[K,N] (this rank's partial over all M rows).  Rows owned by
 * `rank` ([rank*M/world, (rank+1)*M/world)) are folded in the epilogue:
 *   output = bf16( P_owned + sum_{p<world-1} peer_recv[p] )   (fp32 adds)
 * after acquire-waiting the flags of each peer tile; every other row is the
 * would-be send and is written to workspace.  The producer role copies
 * peer_src into peer_recv tile by tile and release-stores the flags.
 * Replaces gemm_rs_multinode::entrypoint_fused
 * (reference include/operators/gemm_rs/gemm_rs.cuh:510-935): compute_tile_impl
 * (src/gemm_rs.cu:36-114) + reduce_tiles_ws (src/gemm_rs.cu:685-845). */
typedef struct mk_gemm_rs_args {
  const void* A;          /* bf16 [M, K] */
  const void* B;          /* bf16 [K, N] */
  void* workspace;        /* bf16 [M, N]; non-owned rows written */
  void* output;           /* bf16 [M/world, N] owned slice */
  const void* peer_src;   /* bf16 [world-1, M/world, N] partials to stage */
  void* peer_recv;        /* bf16 [world-1, M/world, N] staged partials */
  int64_t M, N, K;
  int32_t world, rank;
  uint32_t* flags;              /* [(world-1) * (M/world)/128] */
  const int32_t* stage_order;   /* [(world-1) * (M/world)/128]; NULL = ascending */
  uint32_t epoch;
  int32_t gated;
  int32_t num_producers;        /* as in mk_ag_gemm; -1 and -2 = cooperative staging, even share;
                                   <= -3 = co-resident staging kernel (needs split_ws) */
  int32_t num_cus;
  uint32_t spin_limit;
  uint32_t* error_word;
  uint32_t* stage_counters;     /* [(world-1) * (M/world)/128] for producers == -1 */
  void* split_ws;          /* optional K-split workspace (see mk_query_workspace_bytes);
                              zero-filled before its first use, left zeroed by every
                              launch; NULL = no K-split of the tail round */
  int64_t split_ws_bytes;
  /* Optional device word holding the epoch: when set, the launch reads the
   * epoch from it (never 0) instead of `epoch`, so a HIP graph that records
   * mk_epoch_advance and this launch gates every replay on a new epoch with
   * no host work.  NULL = use `epoch`. */
  const uint32_t* epoch_ptr;
} mk_gemm_rs_args;
int mk_gemm_rs(const mk_gemm_rs_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* GEMM + all-reduce at one rank's share.
 *   C_final = bf16( A @ B + sum_{p < world-1} peer_recv[p] )   (fp32 adds, p ascending)
 * over all M rows: the reduce epilogue of mk_gemm_rs with every row owned.
 * The producer role (or cooperative staging, num_producers = -1) copies
 * peer_src into peer_recv in 128-row blocks, flags[(p * M/128) + block] =
 * epoch, in the order stage_order; compute follows the arrival order of each
 * row tile's last peer block.  When done_flags is set, each finished
 * 256x256 output tile t = row_tile * (N/256) + col_tile is published as
 * done_flags[t] = epoch after its bytes are visible at agent scope (the hand-off
 * the reference's broadcast step reads).
 * Replaces gemm_ar_multinode::entrypoint
 * (reference include/operators/gemm_ar/session.cuh:188-215,
 * src/gemm_ar.cu:1-33 compute + intra-AR roles; the reference checks
 * C_final against all_reduce(matmul), bench/gemm_ar_bench.py:510-514). */
typedef struct mk_gemm_ar_args {
  const void* A;          /* bf16 [M, K] */
  const void* B;          /* bf16 [K, N] */
  void* C_final;          /* bf16 [M, N] */
  const void* peer_src;   /* bf16 [world-1, M, N] partials to stage */
  void* peer_recv;        /* bf16 [world-1, M, N] staged partials */
  int64_t M, N, K;
  int32_t world;
  uint32_t* flags;              /* [(world-1) * M/128] */
  const int32_t* stage_order;   /* [(world-1) * M/128]; NULL = ascending, no arrival order */
  uint32_t epoch;
  int32_t gated;
  int32_t num_producers;        /* as in mk_ag_gemm; -1 and -2 = cooperative staging, even share;
                                   <= -3 = co-resident staging kernel (needs split_ws) */
  int32_t num_cus;
  uint32_t spin_limit;
  uint32_t* error_word;
  uint32_t* stage_counters;     /* [(world-1) * M/128] for producers == -1 */
  uint32_t* done_flags;         /* [(M/256) * (N/256)] or NULL */
  void* split_ws;
  int64_t split_ws_bytes;
  /* Optional device word holding the epoch: when set, the launch reads the
   * epoch from it (never 0) instead of `epoch`, so a HIP graph that records
   * mk_epoch_advance and this launch gates every replay on a new epoch with
   * no host work.  NULL = use `epoch`. */
  const uint32_t* epoch_ptr;
} mk_gemm_ar_args;
int mk_gemm_ar(const mk_gemm_ar_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* GEMM + all-reduce at one rank's share, two-shot: this rank reduces only
 * its own row slice and receives the other slices already reduced by their
 * owners (reduce-scatter, then all-gather), so each output row is reduced
 * once across the node — the work split of the reference's multicast
 * all-reduce, where each tile is reduced once for all GPUs
 * (reference src/gemm_ar.cu:9-32, intra-AR role with multimem reduction;
 * include/operators/gemm_ar/session.cuh:188-215).  With s = M/world rows
 * per slice and r = rank:
 *   C_final[r*s .. (r+1)*s)  = bf16( (A @ B)[own rows] + sum_p peer_recv[p] )
 *                              (fp32 adds, p ascending; the reduce epilogue)
 *   C_final[other slices]    = peer_reduced, staged in 128-row blocks
 *   sends[rows outside r's]  = bf16( (A @ B)[those rows] )  (this rank's pushes)
 * One launch: flags / stage_counters / stage_order cover 2*(world-1)*s/128
 * blocks, first the partial blocks of this rank's slice (peer_src ->
 * peer_recv, as mk_gemm_rs), then the reduced blocks (peer_reduced ->
 * C_final, flags[(world-1)*s/128 + b] = epoch once block b is in place).
 * done_flags (optional, [(M/256)*(N/256)]): each finished tile of this rank's
 * slice, as in mk_gemm_ar.  num_producers as in mk_gemm_rs; 0 = everything
 * was staged by someone else (flags published; peer_reduced unread). */
typedef struct mk_gemm_ar2_args {
  const void* A;            /* bf16 [M, K] */
  const void* B;            /* bf16 [K, N] */
  void* C_final;            /* bf16 [M, N] */
  void* sends;              /* bf16 [M, N]; rows outside this rank's slice written */
  const void* peer_src;     /* bf16 [world-1, M/world, N]: peers' partials of this rank's slice, rank order without r */
  void* peer_recv;          /* bf16 [world-1, M/world, N] staged partials */
  const void* peer_reduced; /* bf16 [world-1, M/world, N]: the other slices, reduced, slice order without r */
  int64_t M, N, K;
  int32_t world, rank;
  uint32_t* flags;              /* [2 * (world-1) * (M/world)/128] */
  const int32_t* stage_order;   /* permutation of those blocks; NULL = ascending */
  uint32_t epoch;
  int32_t gated;
  int32_t num_producers;
  int32_t num_cus;
  uint32_t spin_limit;
  uint32_t* error_word;
  uint32_t* stage_counters;     /* [2 * (world-1) * (M/world)/128] */
  uint32_t* done_flags;         /* [(M/256) * (N/256)] or NULL */
  void* split_ws;
  int64_t split_ws_bytes;
  const uint32_t* epoch_ptr;
} mk_gemm_ar2_args;
int mk_gemm_ar_two_shot(const mk_gemm_ar2_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* MoE routing index build (host memory, host CPU).  Restates the reference's
 * host-side builders bench/dispatch_gemm_bench.py:127-188 (build_routing,
 * build_pull_indices) and bench/dispatch_gemm_glu_combine_bench.py:222-293,
 * 513-527 (build_gather_indices, local_rb_per_expert, row_expert) for one
 * rank owning experts [expert_begin, expert_begin + n_local).
 * Rows are grouped by local expert (ascending); inside an expert, source
 * tokens ascend; each expert is padded to a multiple of `row_block` with
 * pull rows (-1,-1,-1).  Tokens come from one source (node 0, dev 0). */
int mk_moe_index_sizes(const int32_t* topk_ids, int32_t num_tokens, int32_t topk,
                       int32_t expert_begin, int32_t n_local, int32_t row_block,
                       int64_t* R_out, int64_t* R_pad_out);

typedef struct mk_moe_index {
  /* all host arrays, caller-allocated */
  int32_t* padded_tokens_per_expert; /* [n_local] */
  int32_t* local_rb_per_expert;      /* [n_local] whole row blocks of real rows */
  int32_t* pull_indices;             /* [R_pad, 3] (src_node, src_dev, src_token) */
  int32_t* row_expert;               /* [R_pad] local expert of each row */
  int32_t* rb_expert;                /* [R_pad / row_block] */
  int32_t* rb_rows;                  /* [R_pad / row_block] real (non-padding) rows per row block */
  float* row_weight;                 /* [R_pad] gate of each row; 0 on padding */
  int32_t* owner_offset;             /* [num_tokens + 1] CSR over source tokens */
  int32_t* row_to_slot;              /* [R_pad] slot of each row; 0 on padding */
  int32_t* row_to_owner;             /* [R_pad] owner dev of each row; -1 on padding */
  int32_t* slot_to_row;              /* [R] inverse of row_to_slot */
} mk_moe_index;
int mk_moe_build_indices(const int32_t* topk_ids, const float* topk_gates,
                         int32_t num_tokens, int32_t topk, int32_t expert_begin,
                         int32_t n_local, int32_t row_block, const mk_moe_index* out);

/* ------------------------------------------------------------------------ */
/* The same routing index tables built on the GPU from top-k ids and gates in
 * device memory (no host round trip), bit-identical to
 * mk_moe_build_indices.  Row tables (pull_indices, row_expert, row_weight,
 * row_to_slot, row_to_owner, slot_to_row) must hold `capacity_rows` rows,
 * rb_expert / rb_rows capacity_rows / row_block entries; R and R_pad land in
 * the device word pair `sizes` when the stream reaches them.  If R_pad >
 * capacity_rows, sizes still reports it and rows past the capacity are not
 * written (capacity_rows = num_tokens * topk + n_local * (row_block - 1)
 * always suffices).  `workspace` holds mk_moe_index_workspace_bytes bytes.
 * At most 4096 local experts.
 * No counterpart in the reference, whose builders are host Python
 * (bench/dispatch_gemm_bench.py:127-188,
 * bench/dispatch_gemm_glu_combine_bench.py:222-293, 511-527). */
typedef struct mk_moe_index_dev_args {
  const int32_t* topk_ids;   /* [num_tokens, topk] device */
  const float* topk_gates;   /* [num_tokens, topk] device */
  int32_t num_tokens, topk, expert_begin, n_local, row_block;
  int64_t capacity_rows;
  void* workspace;
  int64_t workspace_bytes;
  int64_t* sizes;            /* device [2]: R, R_pad */
  mk_moe_index out;          /* device pointers; NULL skips a table */
} mk_moe_index_dev_args;
int64_t mk_moe_index_workspace_bytes(int32_t num_tokens, int32_t topk, int32_t n_local);
int mk_moe_build_indices_dev(const mk_moe_index_dev_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Token permute into expert-contiguous rows:
 *   post[r] = tokens[src_row(r)]   (bit-exact copy), zero on padding rows,
 * src_row = (src_node * devs_per_node + src_dev) * tokens_per_src + src_token.
 * Replaces dispatch_fused (reference src/dispatch_gemm.cu:106-198). */
typedef struct mk_moe_permute_args {
  const void* tokens;           /* bf16 [n_src_rows, H] */
  const int32_t* pull_indices;  /* [R_pad, 3] device */
  void* post_tokens;            /* bf16 [R_pad, H] */
  int64_t R_pad, H;
  int64_t n_src_rows;
  int32_t tokens_per_src, devs_per_node;
  /* Optional device row count {R, R_pad} (the `sizes` pair that
   * mk_moe_build_indices_dev writes), or NULL.  When set, R_pad above is the
   * row capacity the tables and buffers were sized for, and rows at or past
   * sizes[1] are skipped, so the call needs no host read-back of the routed
   * row count (and can be recorded in a HIP graph).  No counterpart in the
   * reference, whose row counts come from its host builders. */
  const int64_t* sizes;
} mk_moe_permute_args;
int mk_moe_permute(const mk_moe_permute_args* args, void* stream);

/* Grouped GEMM over expert-contiguous rows.
 *   mode 0: out[r] = post[r] @ W[e(r)]                 (W: [E, K, N])
 *   mode 1: out[r] = silu(h[:, :I]) * h[:, I:], h = post[r] @ W[e(r)]
 *           (W: [E, K, 2I], out: [R_pad, I])   SwiGLU fused in the epilogue
 * e(r) = rb_expert[r / 128] when rb_expert is given, else the expert whose
 * padded row range [sum_{e'<e} padded[e'], sum_{e'<=e} padded[e']) holds r,
 * from padded_tokens_per_expert (the reference's own table).
 * Replaces group_gemm_fused (reference src/dispatch_gemm.cu:207-408),
 * gemm1_swiglu_fused (src/dispatch_gemm_glu_combine.cu:441-643) and
 * ffn_gemm2/grouped_gemm (src/dispatch_gemm_glu_combine.cu:247-429,647-651). */
typedef struct mk_moe_grouped_gemm_args {
  const void* A;              /* bf16 [R_pad, K] */
  const void* W;              /* bf16 [E, K, Nw] */
  void* out;                  /* bf16 [R_pad, N_out] */
  const int32_t* rb_expert;   /* [R_pad/128] device, or NULL */
  const int32_t* padded_tokens_per_expert; /* [E] device; used when rb_expert is NULL */
  const int32_t* rb_rows;     /* [R_pad/128] real rows per row block, or NULL; lets the
                                 kernel skip MFMAs of all-padding 32-row blocks */
  int64_t R_pad, K, Nw;       /* Nw = W's column count (2I in mode 1) */
  int32_t num_experts;
  int32_t mode;
  int32_t num_cus;
  void* split_ws;              /* optional K-split workspace, as in mk_gemm_args */
  int64_t split_ws_bytes;
  /* Fused dispatch (the reference's moe_dispatch_gemm_fused,
   * include/operators/dispatch_gemm/dispatch_gemm.cuh:238-262): when
   * gather_pull is set, A is the token buffer [n_src_rows, K] and GEMM row r
   * reads token row (src_node * devs_per_node + src_dev) * tokens_per_src +
   * src_token of pull row r (padding rows read zeros); no permuted copy is
   * made.  n_src_rows * K * 2 must stay below 2 GiB. */
  const int32_t* gather_pull;  /* [R_pad, 3] device, or NULL */
  int64_t n_src_rows;
  int32_t tokens_per_src, devs_per_node;
  int32_t tile_n;              /* output tile width: 256, 512 (Nw % 512 == 0), or 0 = library choice */
  /* Optional device {R, R_pad}, as in mk_moe_permute_args: row tiles at or
   * past sizes[1] are not computed (R_pad is the capacity) and the tail
   * round's K-split is planned on the device; the split then needs
   * split_ws to hold mk_query_workspace_bytes() bytes, else it is off. */
  const int64_t* sizes;
} mk_moe_grouped_gemm_args;
int mk_moe_grouped_gemm(const mk_moe_grouped_gemm_args* args, void* stream);

/* Top-k weighted combine back to source-token order (gather, no atomics):
 *   y[t] = sum_{s in [owner_offset[t], owner_offset[t+1])}
 *              row_weight[slot_to_row[s]] * y_expert[slot_to_row[s]]
 * products and sum in fp32; output fp32 (out_dtype 0) or bf16 (1).
 * y_expert, row_weight and slot_to_row are read only inside owner_offset's
 * ranges, so with no routed rows they may be NULL (then y = 0).  Every MoE
 * entry accepts R_pad == 0 (no rows routed to this rank): permute and the
 * grouped GEMMs do nothing and need no buffers.
 * Replaces combine_producer_fused + combine_gather_owner
 * (reference src/dispatch_gemm_glu_combine.cu:736-818). */
typedef struct mk_moe_combine_args {
  const void* y_expert;         /* bf16 [R_pad, H] */
  const float* row_weight;      /* [R_pad] */
  const int32_t* owner_offset;  /* [num_tokens + 1] */
  const int32_t* slot_to_row;   /* [R] */
  void* y_out;                  /* [num_tokens, H] fp32 or bf16 */
  int64_t num_tokens, H;
  int32_t out_dtype;
} mk_moe_combine_args;
int mk_moe_combine(const mk_moe_combine_args* args, void* stream);

/* Turns the reference's producer-side tables (row_to_slot, row_to_owner;
 * bench/dispatch_gemm_glu_combine_bench.py:264-279) into the gather table
 * the combine reads: slot_to_row[0 .. slot_capacity) is first set to -1,
 * then slot_to_row[row_to_slot[r]] = r for every row r with
 * row_to_owner[r] == owner.  Rows of other owners (another GPU combines
 * them) are left out, and the combine skips slots that stay -1.  A slot
 * outside [0, slot_capacity) is not written; it sets bit 1 of *error_word
 * when error_word is non-NULL. */
int mk_moe_invert_slots(const int32_t* row_to_slot, const int32_t* row_to_owner, int64_t R_pad, int32_t owner,
                        int64_t slot_capacity, int32_t* slot_to_row, uint32_t* error_word, void* stream);

/* rb_rows[b] = number of rows r in [128b, 128b+128) with pull_indices[r][0] >= 0
 * (device, from the reference's pull table). */
int mk_moe_tile_rows(const int32_t* pull_indices, int64_t R_pad, int32_t* rb_rows, void* stream);

/* The whole local MoE layer in one call: permute -> grouped GEMM1 + SwiGLU ->
 * grouped GEMM2 -> combine (four launches on `stream`).
 * Replaces moe_dispatch_gemm_glu_combine_fused
 * (reference include/operators/dispatch_gemm_glu_combine/dispatch_gemm_glu_combine.cuh:307-548). */
typedef struct mk_moe_ffn_args {
  const void* tokens;           /* bf16 [n_src_rows, H] */
  const int32_t* pull_indices;  /* [R_pad, 3] */
  const int32_t* rb_expert;     /* [R_pad/128], or NULL */
  const int32_t* padded_tokens_per_expert; /* [E]; used when rb_expert is NULL */
  const int32_t* rb_rows;       /* [R_pad/128] real rows per row block, or NULL */
  const float* row_weight;      /* [R_pad] */
  const int32_t* owner_offset;  /* [num_tokens + 1] */
  const int32_t* slot_to_row;   /* [R] */
  const void* w1;               /* bf16 [E, H, 2I] (gate | up) */
  const void* w2;               /* bf16 [E, I, H] */
  void* post_tokens;            /* bf16 [R_pad, H]  (caller scratch / output) */
  void* act;                    /* bf16 [R_pad, I] */
  void* y_expert;               /* bf16 [R_pad, H] */
  void* y_out;                  /* [num_tokens, H] fp32 or bf16 */
  int64_t num_tokens, n_src_rows, R_pad, H, I;
  int32_t num_experts;
  int32_t tokens_per_src, devs_per_node;
  int32_t out_dtype;
  int32_t num_cus;
  void* split_ws;              /* optional K-split workspace, as in mk_gemm_args */
  int64_t split_ws_bytes;
  int32_t fuse_dispatch;       /* 1: GEMM1 gathers tokens itself, post_tokens is not written */
  int32_t tile_n;              /* grouped GEMM tile width, as in mk_moe_grouped_gemm_args */
  /* Optional device {R, R_pad}, as in mk_moe_permute_args: with it the
   * whole layer (permute, both grouped GEMMs, combine) runs from the device
   * tables of mk_moe_build_indices_dev at their capacity, with no host
   * read-back between the index build and the combine. */
  const int64_t* sizes;
} mk_moe_ffn_args;
int mk_moe_ffn_combine(const mk_moe_ffn_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* K-split workspace size.  When the output tiles do not fill the last round
 * of the persistent grid (tiles % compute workgroups != 0), the GEMM entry
 * points split each tile of that tail round along K over 2-4 workgroups;
 * the parts exchange fp32 partial tiles and ready flags through `split_ws`.
 * This returns the bytes `split_ws` needs on the current device for any
 * shape and grid (4 KB of flag words plus one 256x256 fp32 tile per CU); `which`, M,
 * N and K are accepted for symmetry and do not change the answer.  A
 * workspace serves one launch at a time: launches that share it must be
 * ordered (same stream).  No counterpart in the reference, whose tail round
 * simply idles (src/ag_gemm.cu:265-461). */
int64_t mk_query_workspace_bytes(int32_t which, int64_t M, int64_t N, int64_t K);

/* Diagnostic, no counterpart in the reference (its benches price against
 * the published peak only): the MFMA throughput ceiling of the device under
 * sustained load.  num_wg workgroups of mk_probe_threads() threads each run
 * `iters` iterations of 16 independent v_mfma_f32_32x32x16_bf16 per wave
 * (32768 FLOP each) on random bf16 operands, no memory traffic.
 * sink: fp32 [num_wg * mk_probe_threads()] (keeps the work live);
 * clocks: u64 [num_wg * 2] = per workgroup (shader clock cycles, 100 MHz
 * constant-clock ticks) around the loop, whose ratio gives the engine clock
 * the matrix cores ran at.  Used by bench.py next to the roofline. */
int mk_probe_mfma_ceiling(int64_t iters, int32_t num_wg, float* sink, uint64_t* clocks, void* stream);
int32_t mk_probe_threads(void);

/* Number of compute units of the current device (0 if no device). */
int32_t mk_device_cu_count(void);

const char* mk_last_error_string(void);

/* Advances a device epoch word on the stream: *epoch_ptr += 1, skipping 0
 * (the value flags start at).  Recorded in a HIP graph before gated launches
 * that read epoch_ptr, it gives each replay a new epoch.  Device-side
 * counterpart of the reference's host epoch helpers (set_epoch /
 * prepare_epoch / commit_epoch, include/operators/ag_gemm/session.cuh:192-230). */
int mk_epoch_advance(uint32_t* epoch_ptr, void* stream);

/* ABI version, bumped on any signature change (2: split_ws fields; 4: MoE
 * `sizes`; 5: epoch_ptr; 6: mk_ag_gemm n_present, mk_moe_invert_slots owner
 * and slot capacity). */
int32_t mk_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MK_H_ */
