// mk_gemm.hip — persistent, tile-scheduled bf16 GEMM for gfx950 with
// workgroup roles:
//   * producer workgroups (blockIdx.x < n_prod) stage 128-row tiles of HBM
//     data (AllGather shards or peer partials) and release-store a flag per
//     tile — the in-GPU stand-in for the reference's intra_comm_sm gather
//     (reference src/ag_gemm.cu:31-215);
//   * compute workgroups run BM x BN output tiles (BN = 256; 512 for the
//     128-row expert tiles of the grouped GEMMs) on
//     v_mfma_f32_32x32x16_bf16, optionally acquire-waiting the A-row flags
//     before a tile (reference src/ag_gemm.cu:374-377) and optionally folding
//     staged peer partials into the epilogue (reference src/gemm_rs.cu:685-845
//     reduce_tiles_ws, here in fp32 with a single rounding).
//
// Operands: A row-major [M,K]; B row-major [K,N], the layout the reference
// keeps its weights in (bench/dispatch_gemm_glu_combine_bench.py:546-553).
//
// Pipeline.  Both operands go HBM -> LDS with buffer_load_dwordx4 ... lds
// (no VGPR staging) through an S-deep ring of 32-deep K stages:
//   A stage: BM rows x 64 B, K-contiguous; 16-byte unit c of row r lives at
//            unit c ^ ((r >> 2) & 3), so MFMA operand reads (ds_read_b128,
//            16 consecutive rows per 16-lane group) are bank-conflict free;
//   B stage: 32 k-rows x 2*BN B, N-contiguous exactly as B is stored; unit c
//            of k-row k lives at c ^ (4 * (k & 3)).  MFMA B operands are read
//            with ds_read_b64_tr_b16: inside each 16-lane group, lane 4j+q
//            supplies 4 columns of k-row j and every lane receives one column
//            across the 4 k-rows, so B needs no transpose pass at all.
// The MFMA is issued as (B-fragment, A-fragment), so each lane's accumulator
// holds 4 consecutive N values of one row and the epilogue writes 8-byte row
// segments.  Workgroups have 4 waves (one per SIMD, 128x128 wave tiles) or 8
// waves (two per SIMD, 128x64 wave tiles: one wave's stalls are covered by
// the other's MFMAs).
#include "mk_device.h"
#include "mk_internal.h"
#include "mk_once.h"
#include <mutex>
#include <vector>

namespace mk {

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Tile configuration
// ---------------------------------------------------------------------------
template <int BM_, int WAVES_, int BN_ = 256>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WAVES = WAVES_, NT = 64 * WAVES_;
  static constexpr int WM = 2, WN = WAVES_ / 2;             // wave grid
  static constexpr int WTM = BM / WM, WTN = BN / WN;        // wave tile
  static constexpr int FM = WTM / 32, FN = WTN / 32;        // 32x32 blocks per wave
  static constexpr int BKD = 32;                            // K per stage
  static constexpr uint32_t A_BYTES = BM * BKD * 2;         // BM x 64 B
  static constexpr uint32_t BROW = BN * 2;                  // bytes per LDS B k-row
  static constexpr uint32_t B_BYTES = BKD * BROW;           // 32 k-rows
  static constexpr int B_UPR = BN / 8;                      // 16-byte units per B k-row
  static constexpr uint32_t STAGE = A_BYTES + B_BYTES;
  // Schedule tables in static LDS (arrival-ordered tile order, cooperative
  // staging): only the 256-row kernels (AllGather / reduce-scatter /
  // all-reduce) use them; the 128-row expert kernels give the LDS to the ring.
  static constexpr bool kSched = (BM == 256);
  // ring depth: as deep as the 160 KB LDS allows (next to the static tables
  // where there are any): 4 x 40 KB for the 128 x 512 expert tiles
  static constexpr int S = (BN == 512) ? 4 : (BM == 256) ? 4 : 6;
  static constexpr uint32_t LDS_BYTES = S * STAGE;
  static constexpr int A_INST = A_BYTES / 1024 / WAVES_;    // DMA instructions per wave per stage
  static constexpr int B_INST = B_BYTES / 1024 / WAVES_;
  static constexpr int LOADS = A_INST + B_INST;             // vmcnt per stage
  static_assert(A_INST >= 1 && B_INST >= 1, "tile too small for the wave count");
  static_assert(FM >= 1 && FN >= 2 && FN % 2 == 0, "wave tile");
};

// ---------------------------------------------------------------------------
// Tile decode
// ---------------------------------------------------------------------------

// Grouped ("super-M") order: runs of group_m row tiles are walked
// column-major so concurrently running workgroups share A rows and B columns
// (reference src/ag_gemm.cu:230-253 uses SUPER_M=12 for the same purpose).
__device__ __forceinline__ void decode_grouped(int t, int tiles_m, int tiles_n, int group_m,
                                               int& tm, int& tn) {
  const int group = group_m * tiles_n;
  const int g = t / group;
  const int first = g * group_m;
  const int gm = min(tiles_m - first, group_m);
  const int r = t - g * group;
  tm = first + r % gm;
  tn = r / gm;
}

// Global column of B for LDS B-column q (q a multiple of 8).  With the SwiGLU
// epilogue a 256-column tile holds 128 gate columns (LDS columns 0..127:
// gate columns tn*128 ..) and the 128 matching up columns (LDS 128..255:
// I + tn*128 ..), so every B k-row is fetched as two 256-byte segments.
// Wave wn's fragments read the LDS blocks b_block gives, so fragment jb and
// jb + FN/2 of one thread hold a gate and its up column.
template <class C, int EPI>
__device__ __forceinline__ int b_col(const GemmKParams& p, int tn, int q) {
  if constexpr (EPI == kEpiSwiGLU) {
    constexpr int half = C::BN / 2;
    return q < half ? tn * half + q : p.swiglu_I + tn * half + (q - half);
  } else {
    return tn * C::BN + q;
  }
}

// 32-column LDS block that wave wn's B fragment jb reads.  With SwiGLU the
// wave's gate fragments (jb < FN/2) are adjacent blocks of the gate half and
// its up fragments the same blocks of the up half, so fragment jb and
// jb + FN/2 of one thread hold a gate column and its up column, and the
// wave's output columns are contiguous.
template <class C, int EPI>
__device__ __forceinline__ int b_block(int wn, int jb) {
  if constexpr (EPI == kEpiSwiGLU) {
    constexpr int H = C::FN / 2;
    return jb < H ? wn * H + jb : C::WN * H + wn * H + (jb - H);
  } else {
    return wn * C::FN + jb;
  }
}

// Epoch of this launch: the device word when the caller passed one (it was
// written by an earlier launch on the stream, so it is visible and fixed for
// the whole launch), else the launch argument.
__device__ __forceinline__ uint32_t launch_epoch(const GemmKParams& p) {
  return p.epoch_ptr
             ? __builtin_amdgcn_readfirstlane(__hip_atomic_load(p.epoch_ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
             : p.epoch;
}

// ---------------------------------------------------------------------------
// Producer role: copy 128-row blocks src -> dst in stage order, then publish.
// ---------------------------------------------------------------------------
// Source and destination of staged block b (see st_split_at).
__device__ __forceinline__ void stage_block(const GemmKParams& p, int b, const uint16_t*& src, uint16_t*& dst) {
  const int64_t block_elems = (int64_t)kFlagRows * p.st_cols;
  if (p.st_src2 && b >= p.st_split_at) {
    const int b2 = b - p.st_split_at;
    src = p.st_src2 + (int64_t)b2 * block_elems;
    dst = p.st_dst2 + (int64_t)(b2 + (b2 >= p.st_dst2_skip_at ? p.st_dst2_skip : 0)) * block_elems;
  } else {
    src = p.st_src + (int64_t)b * block_elems;
    dst = p.st_dst + (int64_t)b * block_elems;
  }
}

template <int NT>
__device__ void producer_role(const GemmKParams& p, int pid) {
  const int64_t block_elems = (int64_t)kFlagRows * p.st_cols;
  for (int i = pid; i < p.st_nblocks; i += p.n_prod) {
    const int b = p.st_order ? p.st_order[i] : i;
    const uint16_t* src;
    uint16_t* dst;
    stage_block(p, b, src, dst);
    if (i >= p.st_present) copy_wt<NT, 16>(src, dst, block_elems / 8);
    // every wave's write-through stores performed, then one publication
    wait_vmem_all();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(p.st_flags + b, launch_epoch(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// One staging piece: global piece q is piece q % kPieces of the 128-row
// block at stage position q / kPieces.  Copied by the NT threads that call
// this (U loads in flight per thread); blocks at the first st_present
// positions are already in place (this rank's own shard) and are counted and
// published without a copy.  Returns the piece's block.
template <int NT, int U>
__device__ __forceinline__ int stage_piece(const GemmKParams& p, int q) {
  const int64_t block_elems = (int64_t)kFlagRows * p.st_cols;
  const int64_t piece_vec = block_elems / 8 / kPieces;  // 16-byte units per piece
  const int pos = q / kPieces, piece = q % kPieces;
  const int b = p.st_order ? p.st_order[pos] : pos;
  const uint16_t* src;
  uint16_t* dst;
  stage_block(p, b, src, dst);
  const int64_t off = (int64_t)piece * piece_vec * 8;
  if (pos >= p.st_present) copy_wt<NT, U>(src + off, dst + off, piece_vec);
  return b;
}

// One finished piece of block b (its stores performed at agent scope by
// every thread that made them): bump the block's counter; the increment
// that completes the block publishes the block's flag.  The increments form
// one chain per block, so a relaxed agent-scope flag store suffices.
// Counters are never reset: completion is detected modulo kPieces.
__device__ __forceinline__ void count_piece(const GemmKParams& p, int b) {
  const uint32_t old = __hip_atomic_fetch_add(p.st_counters + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old % kPieces == kPieces - 1)
    __hip_atomic_store(p.st_flags + b, launch_epoch(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cooperative staging: every compute workgroup copies its share of the
// staging pieces (a workgroup copies pieces q, q + stride, ... — stride
// n_cons when every workgroup shares a range, the group size when one half
// of the grid does).  A workgroup stages in increasing q and may stop at any
// limit and resume later (q and batch are its cursor), which lets the copy
// run between tile rounds instead of all before the first one.
template <int NT>
__device__ void coop_stage(const GemmKParams& p, int stride, int& q, int& batch, int limit) {
  limit = min(limit, p.st_nblocks * kPieces);
  // Pieces are counted in batches of p.st_batch: copy the batch, wait for
  // the stores, one barrier, then count the batch's pieces; the first batch
  // is a single piece so the earliest blocks complete early.
  while (q < limit) {
    int bs[8];
    int n = 0;
    for (; n < batch && q < limit; ++n, q += stride) bs[n] = stage_piece<NT, 16>(p, q);
    wait_vmem_all();
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < n; ++i) count_piece(p, bs[i]);
    batch = p.st_batch;
  }
}

// Claimed staging (st_coop 3), the compute workgroups' side: pieces are
// handed out in stage order through the launch's claim word (st_claim[0]),
// which the co-resident staging kernel (stage_kernel) draws from one piece
// at a time.  Before a tile round, a workgroup that finds pieces below
// `need` (what the round waits for) still unclaimed claims its 1/n_cons
// share of them and copies it; when the staging kernel is ahead, it copies
// nothing.  The claim word starts every launch at zero: each claimer
// (staging wave or compute workgroup) bumps st_claim[1] once it will claim
// no more, and the last of them zeroes both words for the next launch.
template <int NT>
__device__ void claim_stage(const GemmKParams& p, int need, int n_cons, int* sh) {
  const int total = p.st_nblocks * kPieces;
  need = min(need, total);
  if (threadIdx.x == 0) {
    const int done = (int)__hip_atomic_load(p.st_claim, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int first = 0, n = 0;
    if (done < need) {
      const int share = (need - done + n_cons - 1) / n_cons;
      first = (int)__hip_atomic_fetch_add(p.st_claim, (uint32_t)share, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      n = max(0, min(share, total - first));
    }
    sh[0] = first;
    sh[1] = n;
  }
  __syncthreads();
  const int first = sh[0], n = sh[1];
  __syncthreads();  // sh is free again
  for (int i0 = 0; i0 < n; i0 += 8) {
    int bs[8];
    const int m = min(8, n - i0);
    for (int i = 0; i < m; ++i) bs[i] = stage_piece<NT, 16>(p, first + i0 + i);
    wait_vmem_all();
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) count_piece(p, bs[i]);
  }
}

// A claimer that will claim no more pieces in this launch checks out; the
// last of the `participants` zeroes the claim word and the check-out count.
__device__ __forceinline__ void claim_checkout(const GemmKParams& p, uint32_t participants) {
  if (__hip_atomic_fetch_add(p.st_claim + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == participants - 1) {
    __hip_atomic_store(p.st_claim, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p.st_claim + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The co-resident staging kernel: one-wave workgroups that copy pieces in
// stage order, drawing one piece at a time from the claim word (the next
// claim is issued before the current piece's copy, so its latency hides
// behind the copy), and count/publish each piece like the compute
// workgroups do.  64 VGPRs and no LDS: the register-capped GEMM leaves that
// room on every SIMD, so these waves run beside the GEMM's workgroups — the
// copy overlaps the MFMA work instead of taking turns with it (reference:
// the intra_comm_sm copy of src/ag_gemm.cu:49-83 running beside
// fused_comp_sm, :265-461).
__global__ __launch_bounds__(64) __attribute__((amdgpu_num_vgpr(32))) void stage_kernel(GemmKParams p) {
  const int total = p.st_nblocks * kPieces;
  int c = 0;
  if (threadIdx.x == 0) c = (int)__hip_atomic_fetch_add(p.st_claim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c = __builtin_amdgcn_readfirstlane(c);
  while (c < total) {
    int next = 0;
    if (threadIdx.x == 0)
      next = (int)__hip_atomic_fetch_add(p.st_claim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int b = stage_piece<64, 8>(p, c);
    wait_vmem_all();  // this wave's stores are performed at agent scope
    if (threadIdx.x == 0) count_piece(p, b);
    c = __builtin_amdgcn_readfirstlane(next);
  }
  if (threadIdx.x == 0) claim_checkout(p, gridDim.x + p.st_claimers);
}

// ---------------------------------------------------------------------------
// LDS-DMA helpers
// ---------------------------------------------------------------------------

// Raw buffer descriptor (gfx9 word 3) for inline-asm buffer instructions.
__device__ __forceinline__ u32x4_t make_rsrc_v(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000u;
  return r;
}

// 16-byte buffer load straight into LDS: lane l's 16 bytes land at
// lds_addr + 16*l.  Issued through inline asm so the compiler does not
// serialise every later LDS read behind it; completion is tracked by hand
// with wait_stage (vmcnt) followed by a workgroup barrier.
// The compiler's hazard pass does not look inside inline asm, so the wait
// states are written here: a VMEM instruction that reads an SGPR written by a
// VALU instruction (v_readlane / v_readfirstlane, e.g. a reloaded SGPR spill)
// needs 5 wait states, and an LDS DMA after an SALU write of M0 needs 1.
// Without them the load can use a stale rsrc / soffset and fetch wrong bytes.
// M0 is listed as clobbered; the compiler reports that it does not preserve
// a reserved register across inline asm, so it must hold nothing live here.
// In the generated code the compiler's own M0 uses (v_writelane lane
// selects in atomic expansions) set M0 immediately before the use, with no
// DMA between.
__device__ __forceinline__ void dma16(u32x4_t r, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}

// Two LDS DMAs in one asm statement (nothing can be scheduled between them),
// so the 5-wait-state guard is paid once per pair.
__device__ __forceinline__ void dma16x2(u32x4_t r, uint32_t lds0, uint32_t lds1, uint32_t v0, uint32_t v1,
                                        uint32_t soff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %2, %4, %5 offen lds\n\t"
      "s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %3, %4, %5 offen lds"
      :
      : "s"(lds0), "s"(lds1), "v"(v0), "v"(v1), "s"(r), "s"(soff)
      : "memory", "m0");
}

// N DMAs into consecutive 1 KB LDS blocks starting at lds, paired.
template <int N>
__device__ __forceinline__ void dma16_run(u32x4_t r, uint32_t lds, const uint32_t (&voff)[N], uint32_t soff) {
#pragma unroll
  for (int i = 0; i + 1 < N; i += 2) dma16x2(r, lds + i * 1024, lds + (i + 1) * 1024, voff[i], voff[i + 1], soff);
  if constexpr (N % 2) dma16(r, lds + (N - 1) * 1024, voff[N - 1], soff);
}

// s_waitcnt vmcnt(n) (n <= 63), other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until at most `pending` of this thread's most recent stages (L DMA
// instructions each) are still in flight, i.e. every older stage has landed.
template <int S, int L>
__device__ __forceinline__ void wait_stage(int pending) {
  static_assert(S <= 7 && (S - 1) * L < 64, "ring too deep for the waitcnt ladder");
  if (pending >= 5 && S > 5) { wait_vm<(S > 5 ? 5 * L : 0)>(); return; }
  if (pending >= 4 && S > 4) { wait_vm<(S > 4 ? 4 * L : 0)>(); return; }
  if (pending >= 3 && S > 3) { wait_vm<(S > 3 ? 3 * L : 0)>(); return; }
  if (pending >= 2 && S > 2) { wait_vm<2 * L>(); return; }
  if (pending >= 1) { wait_vm<L>(); return; }
  wait_vm<0>();
}

__device__ __forceinline__ bf16x4_t lds_tr4(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (__attribute__((address_space(3))) bf16x4_t*)((__attribute__((address_space(3))) char*)(p)));
}

// ---------------------------------------------------------------------------
// Epilogue of one BM x BN tile.  acc[i][j][4a+b] is C[m][n] with
// m = m0 + wm*WTM + 32i + ml and n (in tile) = wn*WTN + 32j + 8a + 4kg + b.
// ---------------------------------------------------------------------------
// s_waitcnt lgkmcnt(0), other counters untouched (gfx9 encoding).
__device__ __forceinline__ void wait_lgkm_all() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Row-major store of a wave's WTM x WTN bf16 sub-tile through a private LDS
// region.  The accumulator layout gives each lane 4 consecutive columns of
// one row, so a direct store instruction touches 32 rows with 16 bytes each:
// a 128 KB tile became ~1000 partial-line L2 writes per wave, and the tile
// epilogue took 13 us of a 200 us tile.  Here each 32-row block goes to LDS
// as rows of WTN bf16 (row pitch padded by 16 bytes, so the 8-byte writes of
// the 32 rows spread over the banks), then comes back 16 bytes per lane
// with consecutive lanes along a row: every store instruction writes whole
// WTN*2-byte row segments.  The region is the wave's own, so only this
// wave's LDS ordering matters (lgkmcnt waits); the caller's workgroup
// barrier must precede the next use of the ring.
template <class C, int NJ = C::FN, bool NT = false>
__device__ __forceinline__ void store_rows(uint16_t* base, int64_t ldc, f32x16 (&acc)[C::FM][C::FN], char* smem,
                                           int wave, int lane) {
  constexpr int W = NJ * 32;              // columns stored per row: accumulator blocks j < NJ
  constexpr int PITCH = W * 2 + 16;       // bytes per LDS row
  constexpr int LPR = W * 2 / 16;         // lanes per row (16 bytes each)
  constexpr int RPI = 64 / LPR;           // rows per store instruction
  static_assert(64 % LPR == 0 && 32 % RPI == 0, "store_rows shape");
  // The lane index goes through an empty asm so that nothing derived from
  // it is hoisted above the K loop (it would stay live across the loop and
  // push the loop's operand registers into spills).
  int l = lane;
  asm volatile("" : "+v"(l));
  const int ml = l & 31, kg = l >> 5;
  char* reg = smem + wave * 32 * PITCH;
  const int rr = l / LPR, cc = l % LPR;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        uint2 w;
        w.x = pack_bf16x2(acc[i][j][4 * a + 0], acc[i][j][4 * a + 1]);
        w.y = pack_bf16x2(acc[i][j][4 * a + 2], acc[i][j][4 * a + 3]);
        *reinterpret_cast<uint2*>(reg + ml * PITCH + (32 * j + 8 * a + 4 * kg) * 2) = w;
      }
    wait_lgkm_all();
#pragma unroll
    for (int r = 0; r < 32 / RPI; ++r) {
      const int row = r * RPI + rr;
      const uint4 v = *reinterpret_cast<const uint4*>(reg + row * PITCH + cc * 16);
      uint4* dst = reinterpret_cast<uint4*>(base + (int64_t)(i * 32 + row) * ldc + cc * 8);
      if constexpr (NT) {
        typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(nt_u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_u32x4*>(dst));
      } else {
        *dst = v;
      }
    }
    wait_lgkm_all();  // this block's reads are done before the next block's writes
  }
}

// Reduce epilogue of an owned tile, row-major: each 32-row block of the
// wave's fp32 accumulators goes through the wave's LDS region (rows of WTN
// fp32, pitch padded by 16 bytes) and comes back 8 columns per lane with
// consecutive lanes along a row; the lane then loads the same 8 columns of
// every peer's bf16 partial (16 bytes per peer: whole row segments per
// instruction, 4 peers' loads in flight, the remainder as one more group),
// adds them in rank order in fp32
// (deterministic, one rounding) and stores 16 bytes of the owned output.
// In the accumulator layout every load and store instruction would touch
// 32 rows with 8 bytes each.
template <class C>
__device__ __forceinline__ void reduce_rows(const GemmKParams& p, f32x16 (&acc)[C::FM][C::FN], int lrow0, int col0,
                                            char* smem, int wave, int lane) {
  constexpr int PITCH = C::WTN * 4 + 16;  // bytes per LDS row (fp32)
  constexpr int LPR = C::WTN / 8;         // lanes per row (8 columns each)
  constexpr int RPI = 64 / LPR;           // rows per instruction
  constexpr int kPeers = 4;               // peer loads in flight per lane
  static_assert(64 % LPR == 0 && 32 % RPI == 0, "reduce_rows shape");
  int l = lane;
  asm volatile("" : "+v"(l));  // keep lane-derived addressing below the K loop
  const int ml = l & 31, kg = l >> 5;
  char* reg = smem + wave * 32 * PITCH;
  const int rr = l / LPR, cc = l % LPR;
  const int64_t peer_stride = (int64_t)p.rs_own_rows * p.ldc;
  const int np = p.rs_npeers;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 w;
#pragma unroll
        for (int b = 0; b < 4; ++b) w[b] = acc[i][j][4 * a + b];
        *reinterpret_cast<f32x4*>(reg + ml * PITCH + (32 * j + 8 * a + 4 * kg) * 4) = w;
      }
    wait_lgkm_all();
    for (int r = 0; r < 32 / RPI; ++r) {
      const int row = r * RPI + rr;
      const f32x4 lo = *reinterpret_cast<const f32x4*>(reg + row * PITCH + cc * 32);
      const f32x4 hi = *reinterpret_cast<const f32x4*>(reg + row * PITCH + cc * 32 + 16);
      float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      const uint16_t* src = p.rs_recv + (int64_t)(lrow0 + i * 32 + row) * p.ldc + col0 + cc * 8;
      int q = 0;
      for (; q + kPeers <= np; q += kPeers) {
        uint4 v[kPeers];
#pragma unroll
        for (int u = 0; u < kPeers; ++u) v[u] = *reinterpret_cast<const uint4*>(src + (q + u) * peer_stride);
#pragma unroll
        for (int u = 0; u < kPeers; ++u) {
          x[0] += bf16_lo(v[u].x); x[1] += bf16_hi(v[u].x);
          x[2] += bf16_lo(v[u].y); x[3] += bf16_hi(v[u].y);
          x[4] += bf16_lo(v[u].z); x[5] += bf16_hi(v[u].z);
          x[6] += bf16_lo(v[u].w); x[7] += bf16_hi(v[u].w);
        }
      }
      if (q < np) {
        // the last np - q peers as one more group in flight (indices
        // clamped to the last peer, so no branch splits the loads)
        uint4 v[kPeers];
#pragma unroll
        for (int u = 0; u < kPeers; ++u)
          v[u] = *reinterpret_cast<const uint4*>(src + (int64_t)min(q + u, np - 1) * peer_stride);
#pragma unroll
        for (int u = 0; u < kPeers; ++u)
          if (q + u < np) {
            x[0] += bf16_lo(v[u].x); x[1] += bf16_hi(v[u].x);
            x[2] += bf16_lo(v[u].y); x[3] += bf16_hi(v[u].y);
            x[4] += bf16_lo(v[u].z); x[5] += bf16_hi(v[u].z);
            x[6] += bf16_lo(v[u].w); x[7] += bf16_hi(v[u].w);
          }
      }
      uint4 o;
      o.x = pack_bf16x2(x[0], x[1]); o.y = pack_bf16x2(x[2], x[3]);
      o.z = pack_bf16x2(x[4], x[5]); o.w = pack_bf16x2(x[6], x[7]);
      typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
      __builtin_nontemporal_store(nt_u32x4{o.x, o.y, o.z, o.w},
                                  reinterpret_cast<nt_u32x4*>(p.rs_out + (int64_t)(lrow0 + i * 32 + row) * p.ldc +
                                                              col0 + cc * 8));
    }
    wait_lgkm_all();  // this block's reads are done before the next block's writes
  }
}

template <class C, int EPI>
__device__ __forceinline__ void store_tile(const GemmKParams& p, f32x16 (&acc)[C::FM][C::FN], int m0, int tn,
                                           int tid, char* smem) {
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WN, wn = wave % C::WN;
  if constexpr (EPI == kEpiStore) {
    // the 128-row expert tiles write rows read by a later kernel (GEMM2's
    // y_expert by the combine): nontemporal stores, which measured faster
    // for both (config 5: GEMM2 224 -> 211 us, layer -6 us)
    store_rows<C, C::FN, C::BM == 128>(p.C + (int64_t)(m0 + wm * C::WTM) * p.ldc + tn * C::BN + wn * C::WTN, p.ldc,
                                       acc, smem, wave, lane);
    __syncthreads();  // every wave's LDS reads done before the ring is reused
  } else if constexpr (EPI == kEpiSwiGLU) {
    // silu(g) * u in fp32 with silu(g) = g / (1 + e^-g), as the reference
    // computes it (reference src/dispatch_gemm_glu_combine.cu:616-633),
    // in place in the gate accumulators; a wave's gate blocks are adjacent
    // output columns (b_block), so the rows go out as whole segments.
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN / 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float g = acc[i][j][v];
          acc[i][j][v] = (g / (1.0f + __expf(-g))) * acc[i][j + C::FN / 2][v];
        }
    store_rows<C, C::FN / 2, true>(p.C + (int64_t)(m0 + wm * C::WTM) * p.ldc + tn * (C::BN / 2) + wn * (C::WTN / 2),
                                   p.ldc,
                             acc, smem, wave, lane);
    __syncthreads();  // every wave's LDS reads done before the ring is reused
  } else {  // kEpiReduce
    const bool owned = m0 >= p.rs_own_row0 && m0 < p.rs_own_row0 + p.rs_own_rows;
    if (!owned) {
      // the would-be sends: written once, not read here (nontemporal
      // stores measured 854 -> 847 us on config 3)
      store_rows<C, C::FN, true>(p.C + (int64_t)(m0 + wm * C::WTM) * p.ldc + tn * C::BN + wn * C::WTN, p.ldc, acc,
                                 smem, wave, lane);
      __syncthreads();  // every wave's LDS reads done before the ring is reused
    } else {
      const int lr0 = m0 - p.rs_own_row0;  // first row inside the owned slice
      if (p.rs_flags) {
        const int rbs = p.rs_own_rows / kFlagRows;
        constexpr int per = C::BM / kFlagRows;
        if (tid == 0)
          wait_flags<16>([&](int f) { return p.rs_flags + (f / per) * rbs + lr0 / kFlagRows + f % per; },
                     p.rs_npeers * per, launch_epoch(p), p.spin_limit, p.err);
        __syncthreads();
      }
      reduce_rows<C>(p, acc, lr0 + wm * C::WTM, tn * C::BN + wn * C::WTN, smem, wave, lane);
      __syncthreads();  // every wave's LDS reads done before the ring is reused
      if (p.ar_done) {
        // all-reduce: publish the finished tile (the broadcast hand-off).
        // The tile's rows are plain stores, so the flag is a release store:
        // one L2 write-back per tile.
        if (tid == 0) publish_flag(p.ar_done + (m0 / C::BM) * p.tiles_n + tn, launch_epoch(p));
      }
    }
  }
}

// Cursor of a workgroup's cooperative staging between tile rounds.
struct StagePlan {
  const int* round_need;  // per round: last stage position it waits for (null: staged up front)
  int n_rounds;
  int q, batch;           // coop_stage cursor (even-share mode)
  int grp, gid, gsize;    // alternating mode: half of the grid (0/1), id in it, its size (0: even share)
  bool claim;             // claimed mode: before round w, claim a share of what round w needs and is unclaimed
};

// Piece count that rounds 0..r need staged (r = n_rounds: every piece).
__device__ __forceinline__ int need_pieces(const GemmKParams& p, const StagePlan& sp, int r) {
  const int total = p.st_nblocks * kPieces;
  if (r >= sp.n_rounds) return total;
  int need = 0;
  for (int i = 0; i <= r; ++i) need = max(need, (sp.round_need[i] + 1) * kPieces);
  return min(need, total);
}

// Alternating cooperative staging, before whole-tile round w.  Window w
// (before round w) brings the staged pieces up to target(w): at least what
// round w+1 waits for and at least an even share (target(-1): what round 0
// waits for, copied by every workgroup before round 0).  Window w is
// copied by one half of the grid, w % 2, while the other half computes;
// the last window by every workgroup.  128 CUs already saturate HBM with a
// copy, so a half moves a window's pieces about as fast as the whole grid
// would, and each workgroup spends about half as long copying as when every
// workgroup copies before every round.  The halves are XCDs 0-3 and 4-7
// (consumer ids are XCD-major), so tiles sharing an XCD's L2 stay in step.
template <int NT>
__device__ void alt_stage(const GemmKParams& p, int cons_id, StagePlan& sp, int w) {
  const int total = p.st_nblocks * kPieces;
  const int n = sp.n_rounds;
  // Even part of the target: windows 0..n-2 alternate halves (half 0 has
  // h0 = ceil((n-1)/2) of them, half 1 h1 = floor); each half's windows
  // carry equal shares of its half of the pieces left after round 0's, so
  // both halves copy the same amount when the waits do not force more into
  // early windows.
  const int h0 = n / 2, h1 = (n - 1) / 2;
  auto target = [&](int win) {
    if (win < 0) return need_pieces(p, sp, 0);
    if (win >= n - 1) return total;
    const int c0 = win / 2 + 1, c1 = (win + 1) / 2;  // windows 0..win of each half
    const int base = need_pieces(p, sp, 0), rest = total - base;  // pieces after the first window
    const int64_t even = h1 > 0 ? base + ((int64_t)rest * c0 * h1 + (int64_t)rest * c1 * h0) / (2LL * h0 * h1)
                                : (int64_t)total;
    return max(need_pieces(p, sp, win + 1), (int)min<int64_t>(even, total));
  };
  auto copy_range = [&](int lo, int hi, int id, int stride) {
    int q = lo + id, batch = 1;
    coop_stage<NT>(p, stride, q, batch, hi);
  };
  if (w == 0) copy_range(0, target(-1), cons_id, p.n_cons);
  const int lo = target(w - 1), hi = max(lo, target(w));
  if (w == n - 1) copy_range(lo, hi, cons_id, p.n_cons);
  else if (w % 2 == sp.grp) copy_range(lo, hi, sp.gid, sp.gsize);
}

// Partial-sum exchange for K-split tail tiles.  A tile's NT threads hold
// FM*FN*16 fp32 accumulators each; they go to the workspace as 16-byte
// units in register order, unit ((i*FN + j)*4 + a)*NT + tid, so writes and
// reads are fully coalesced and need no layout conversion.  The stores are
// write-through at agent scope (SC1, as in copy_wt).  Buffer
// instructions keep the per-unit offsets in scalar registers (one VGPR of
// addressing in total), which matters: the accumulators already hold most
// of the register file.
template <class C>
__device__ __forceinline__ void put_partial(float* dst, f32x16 (&acc)[C::FM][C::FN], int tid) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(dst, (uint32_t)(C::BM * C::BN * 4));
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 v;
#pragma unroll
        for (int b = 0; b < 4; ++b) v[b] = acc[i][j][4 * a + b];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, tid * 16,
                                               ((i * C::FN + j) * 4 + a) * C::NT * 16, 0x10 /* SC1 */);
      }
}

template <class C>
__device__ __forceinline__ void add_partial(const float* src, f32x16 (&acc)[C::FM][C::FN], int tid, char* smem) {
  // The partial comes in through the (idle) LDS ring by DMA, kChunk units
  // of 16 bytes per thread at a time, two chunks in flight: register-staged
  // loads were limited to 8 in flight per thread by the 128 live
  // accumulators (15 us for a 256 KB partial), the DMA needs no registers.
  // Unit n of thread t sits at (n * NT + t) * 16 in the partial, so a chunk
  // is one contiguous range and each thread reads its own 16-byte slots
  // back (consecutive lanes, consecutive addresses: no bank conflicts).
  constexpr int kUnits = C::FM * C::FN * 4, kChunk = 4, kChunks = kUnits / kChunk;
  constexpr uint32_t CHUNK = kChunk * C::NT * 16;          // bytes per chunk
  constexpr int PER_WAVE = CHUNK / 1024 / C::WAVES;          // 1 KB DMA instructions per wave per chunk
  static_assert(kUnits % kChunk == 0 && PER_WAVE >= 1 && 2 * CHUNK <= C::LDS_BYTES, "add_partial chunks");
  const int lane = tid & 63;
  const uint32_t wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
  const u32x4_t r = make_rsrc_v(src, (uint32_t)(C::BM * C::BN * 4));
  auto issue = [&](int c) {
    const uint32_t buf = lds0 + (uint32_t)(c & 1) * CHUNK;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const uint32_t blk = (wave_u * PER_WAVE + i) * 1024;
      dma16(r, buf + blk, (uint32_t)lane * 16, (uint32_t)c * CHUNK + blk);
    }
  };
  issue(0);
  if (kChunks > 1) issue(1);
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    if (c + 1 < kChunks) wait_vm<PER_WAVE>();  // chunk c landed (chunk c+1 may be in flight)
    else wait_vm<0>();
    __syncthreads();
    const char* buf = smem + (c & 1) * CHUNK;
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int n = c * kChunk + u, i = n / (C::FN * 4), j = (n / 4) % C::FN, a = n % 4;
      const f32x4 v = *reinterpret_cast<const f32x4*>(buf + (u * C::NT + tid) * 16);
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[i][j][4 * a + b] += v[b];
    }
    if (c + 2 < kChunks) {
      wait_lgkm_all();
      __syncthreads();  // every thread is done with this buffer
      issue(c + 2);
    }
  }
  __syncthreads();  // the ring is free again for the epilogue
}

// The fp32 partial of another workgroup added into this thread's
// accumulators, per thread with no workgroup barrier (for a subset of the
// waves): loads in groups of 8, each group's loads issued before its adds.
template <class C>
__device__ __forceinline__ void add_partial_regs(const float* src, f32x16 (&acc)[C::FM][C::FN], int tid) {
  constexpr int kUnits = C::FM * C::FN * 4, kGroup = 8;
  static_assert(kUnits % kGroup == 0, "add_partial_regs grouping");
  const __amdgpu_buffer_rsrc_t r = make_rsrc(src, (uint32_t)(C::BM * C::BN * 4));
#pragma unroll
  for (int g = 0; g < kUnits; g += kGroup) {
    f32x4 v[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u)
      v[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, tid * 16, (g + u) * C::NT * 16, 0));
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int n = g + u, i = n / (C::FN * 4), j = (n / 4) % C::FN, a = n % 4;
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[i][j][4 * a + b] += v[u][b];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---------------------------------------------------------------------------
// Compute role
//
// Work of one consumer: the tiles cons_id, cons_id + n_cons, ... below
// sk_full (whole K each; a partial last round of whole tiles goes to
// consumers spread over the XCDs, xcd_slot), then, when the tile count leaves a partial last
// round (sk_split > 1), one K-split unit of a tail tile: consumer u works on
// tail tile sk_full + u / sk_split, K part u % sk_split.  Parts 1.. write
// fp32 partials to the workspace and release a flag; part 0 acquires the
// flags, adds the partials in part order (deterministic) and runs the
// epilogue.  Every round then keeps all consumers busy.
// ---------------------------------------------------------------------------
// Slot of consumer c among `count` < n_cons slots of a partial round,
// spread evenly over the 8 XCDs (consumer c sits on XCD c / (n_cons / 8)
// after the XCD remap), or -1 when c has none.  Leaving every XCD a few
// idle CUs instead of leaving whole XCDs idle measured faster: an
// 8192x3584x8192 GEMM (448 tiles: one full round + 192 tiles) took 364 us
// against 400 us with the idle CUs on two XCDs (the loaded XCDs clock
// lower).  Which tile a workgroup computes does not change any output bit.
__device__ __forceinline__ int xcd_slot(int c, int n_cons, int count, bool spread) {
  if (!spread || (n_cons & 7) || count >= n_cons) return c < count ? c : -1;
  const int per = n_cons / 8, x = c / per, j = c % per, base = count / 8, rem = count % 8;
  if (j >= base + (x < rem ? 1 : 0)) return -1;
  return x * base + min(x, rem) + j;
}

template <class C, int EPI>
__device__ __forceinline__ void compute_role(const GemmKParams& p, int cons_id, int n_cons, char* smem,
                                             const int* row_perm, const uint16_t* full_list, StagePlan& sp) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / C::WN;
  const int wn = wave % C::WN;
  // Row tiles and tail split from the launch parameters, or from the device
  // row count (tiles past it are not walked; the split follows the rule the
  // host's plan uses: R = tiles % n_cons tail tiles, each split
  // min(4, n_cons / R, K stages / 4) ways when that is at least 2).
  int tiles_m = p.tiles_m, sk_split = p.sk_split, sk_full = p.sk_full;
  if constexpr (C::BM == 128) {
    if (p.rows_dev) {
      const int64_t rows = *p.rows_dev;
      tiles_m = __builtin_amdgcn_readfirstlane((int)min<int64_t>(p.tiles_m, max<int64_t>(rows, 0) / C::BM));
      const int nt = tiles_m * p.tiles_n;
      sk_split = 0;
      sk_full = nt;
      const int R = nt % n_cons;
      if (p.sk_dev && R != 0) {
        const int s = min(min(4, n_cons / R), (p.K / 32) / 4);
        if (s >= 2) {
          sk_split = s;
          sk_full = nt - R;
        }
      }
    }
  }
  const int ntiles = tiles_m * p.tiles_n;
  const int nk_all = p.K / C::BKD;

  // A operand read: row wm*WTM + ml (+32 i), 16-byte unit 2kk + g.
  const int ml = lane & 31, g = lane >> 5;
  uint32_t a_rd[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int row = wm * C::WTM + ml;
    a_rd[kk] = row * 64 + (((2 * kk + g) ^ ((row >> 2) & 3)) << 4);
  }
  // B operand read (transposing): in 16-lane group G, lane 4j+q supplies
  // k-row 8(G/2) + j (+4 for the second half, +16 per K sub-step) and the 4
  // columns 16(G&1) + 4q .. +3 of its 32-column block; after the transpose
  // the lane holds column (lane & 31) of the block for those k-rows.
  const int G = lane >> 4, jr = (lane >> 2) & 3, q = lane & 3;
  uint32_t b_rd[C::FN];
#pragma unroll
  for (int jb = 0; jb < C::FN; ++jb) {
    const int krow = 8 * (G >> 1) + jr;
    const int c = 4 * b_block<C, EPI>(wn, jb) + 2 * (G & 1) + (q >> 1);
    b_rd[jb] = krow * C::BROW + ((c ^ (4 * (krow & 3))) << 4) + (q & 1) * 8;
  }
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
  const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);

  const int full = (sk_split > 1) ? sk_full : ntiles;
  const int n_tail_units = (ntiles - full) * (sk_split > 1 ? sk_split : 0);
  // Whole tiles: rounds 0 .. last_round-1 complete, then a partial round of
  // last_cnt tiles spread over the XCDs.  (The K-split tail units stay in
  // consumer order: spreading them split the grouped order's 8-row-tile
  // runs across XCDs and measured slower on the MoE GEMM1.)
  const int last_cnt = full % n_cons, last_round = full / n_cons;
  const int last_slot = xcd_slot(cons_id, n_cons, last_cnt, p.xcd_remap != 0);
  const int n_full_mine = last_round + (last_slot >= 0 ? 1 : 0);

  // One output tile (or one K range of it): accumulate A[rows] @ B[:, cols]
  // over K stages k0 .. k0+nk into acc.  Called from two places (whole
  // tiles, the K-split unit) so that each call site gets its own register
  // allocation: the partial exchange of the split unit must not raise the
  // register pressure of the whole-tile loop.
  auto tile_body = [&](int t, bool permuted, int k0, int nk, f32x16 (&acc)[C::FM][C::FN], int& m0_out,
                       int& tn_out) __attribute__((always_inline)) {
    int tm, tn;
    if (C::BM == 128 && p.expert_order) {
      // Expert order: tile t lies in the run of row tiles [r0, r1) that
      // share row tile t / tiles_n's expert (tiles t of that run are
      // r0 * tiles_n .. r1 * tiles_n - 1, whatever the order inside it);
      // inside the run, column-major.  A one-tile expert's column tiles
      // are consecutive, so its activation rows are fetched once per XCD;
      // a multi-tile expert's row tiles still stream each weight slice
      // together.  The host sets this only with rb_expert.
      const int rt = __builtin_amdgcn_readfirstlane(t / p.tiles_n);
      const int e = __builtin_amdgcn_readfirstlane(p.rb_expert[rt]);
      // Run bounds 64 row tiles per step: every lane loads one table entry
      // and a ballot finds the first entry of another expert, so a long run
      // (a hot expert) costs one load per 64 tiles, not one per tile.
      const int ln = threadIdx.x & 63;
      int r0 = rt, r1 = rt + 1;
      for (;;) {  // backwards: r0 = one past the last other-expert entry below rt
        const int idx = r0 - 1 - ln;
        const uint64_t other = __ballot(idx < 0 || p.rb_expert[max(idx, 0)] != e);
        if (other) {
          r0 -= __builtin_ctzll(other);  // entries r0-1 .. r0-k share e, entry r0-1-k does not
          break;
        }
        r0 -= 64;
      }
      for (;;) {  // forwards: r1 = the first other-expert entry at or above rt + 1
        const int idx = r1 + ln;
        const uint64_t other = __ballot(idx >= tiles_m || p.rb_expert[min(idx, tiles_m - 1)] != e);
        if (other) {
          r1 += __builtin_ctzll(other);
          break;
        }
        r1 += 64;
      }
      r0 = __builtin_amdgcn_readfirstlane(r0);
      r1 = __builtin_amdgcn_readfirstlane(r1);
      const int local = t - r0 * p.tiles_n, nr = r1 - r0;
      tn = local / nr;
      tm = r0 + local % nr;
    } else {
      decode_grouped(t, tiles_m, p.tiles_n, p.group_m, tm, tn);
    }
    if (permuted) tm = row_perm[tm];
    // Tile coordinates are wave-uniform; keep them scalar.
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    const int m0 = tm * C::BM;

    const uint16_t* Bp = p.B;
    if (p.rb_expert) {
      // clamped like the expert_rows walk: a stale table entry must not
      // form a B base outside the weight tensor
      const int e = __builtin_amdgcn_readfirstlane(min(max(p.rb_expert[tm], 0), p.n_experts - 1));
      Bp += (int64_t)e * p.b_expert_stride;
    } else if (p.expert_rows) {
      // Expert whose padded row range holds row m0 (prefix walk over the
      // per-expert padded counts; E is small).
      int e = 0, end = 0;
      for (; e < p.n_experts; ++e) {
        end += p.expert_rows[e];
        if (m0 < end) break;
      }
      e = __builtin_amdgcn_readfirstlane(min(e, p.n_experts - 1));
      Bp += (int64_t)e * p.b_expert_stride;
    }

    // Row tiles padded past their expert's real rows: each wave skips the
    // MFMAs of its 32-row blocks that hold padding only (their outputs stay
    // zero, as they would be from the zero-filled padding rows).
    int fm_active = C::FM;
    const int rb_real = (C::BM == 128 && p.rb_rows) ? __builtin_amdgcn_readfirstlane(p.rb_rows[tm]) : C::BM;
    if (p.rb_rows) {
      const int real = __builtin_amdgcn_readfirstlane(p.rb_rows[tm]) - wm * C::WTM;
      fm_active = __builtin_amdgcn_readfirstlane(min(max((real + 31) / 32, 0), C::FM));
    }

    // Flag gate on the A rows of this tile (AllGather consumer side).
    if (p.a_flags) {
      if (tid == 0) {
        wait_flags<C::BM / kFlagRows>([&](int f) { return p.a_flags + m0 / kFlagRows + f; }, C::BM / kFlagRows,
                                      launch_epoch(p), p.spin_limit, p.err);
      }
      __syncthreads();
    }

    // Padding rows of a 128-row expert block (rb_rows) get an offset past the
    // buffer's end too: the DMA returns zeros without touching memory.
    // Fused dispatch (grouped GEMMs with gather_pull): A rows are gathered
    // from the token buffer through the pull table — row r of the tile reads
    // token row (src_node * devs + src_dev) * tokens_per_src + src_token;
    // padding rows (src < 0) get an offset past the buffer's end, which the
    // buffer load returns as zeros.
    const u32x4_t rA = p.gather_pull
                           ? make_rsrc_v(p.A, (uint32_t)(p.gather_rows * p.lda * 2))
                           : make_rsrc_v(p.A + (int64_t)m0 * p.lda, (uint32_t)(C::BM * p.lda * 2));
    const u32x4_t rB = make_rsrc_v(Bp, (uint32_t)(p.K * p.ldb * 2));
    // DMA source offsets: lane l of a wave instruction fills LDS unit l of a
    // 1 KB block, i.e. (A) row 16*inst + l/4, unit l%4; (B) k-row
    // (64/B_UPR)*inst + l/B_UPR, unit l%B_UPR.  Each lane fetches the chunk
    // whose swizzled home is that unit.
    uint32_t a_src[C::A_INST], b_src[C::B_INST];
#pragma unroll
    for (int i = 0; i < C::A_INST; ++i) {
      const int row = (wave * C::A_INST + i) * 16 + (lane >> 2);
      const int c = (lane & 3) ^ ((row >> 2) & 3);
      if (C::BM == 128 && p.rb_rows && row >= rb_real) {
        // padding row of an expert block: read as zeros, no memory traffic
        a_src[i] = 0x80000000u;
      } else if (p.gather_pull) {
        const int* pr = p.gather_pull + 3 * (int64_t)(m0 + row);
        const int64_t srow = ((int64_t)pr[0] * p.gather_devs + pr[1]) * p.gather_tps + pr[2];
        a_src[i] = (pr[0] < 0 || pr[2] < 0) ? 0x80000000u : (uint32_t)(srow * p.lda * 2 + c * 16);
      } else {
        a_src[i] = (uint32_t)(row * p.lda * 2 + c * 16);
      }
    }
#pragma unroll
    for (int i = 0; i < C::B_INST; ++i) {
      const int krow = (wave * C::B_INST + i) * (64 / C::B_UPR) + lane / C::B_UPR;
      const int c = (lane % C::B_UPR) ^ (4 * (krow & 3));
      b_src[i] = (uint32_t)(krow * p.ldb * 2 + b_col<C, EPI>(p, tn, c * 8) * 2);
    }
    // Stage kt of this unit is global K stage k0 + kt, kept in ring slot kt % S.
    auto issue = [&](int kt) {
      const uint32_t st = lds_base + (uint32_t)(kt % C::S) * C::STAGE;
      const uint32_t ka = (uint32_t)(k0 + kt) * (C::BKD * 2);
      const uint32_t kb = (uint32_t)(k0 + kt) * (C::BKD * p.ldb * 2);
      dma16_run<C::A_INST>(rA, st + wave_u * C::A_INST * 1024, a_src, ka);
      dma16_run<C::B_INST>(rB, st + C::A_BYTES + wave_u * C::B_INST * 1024, b_src, kb);
    };

#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // Fragment registers: [0] holds the K sub-step kk = 0 operands of a
    // stage, [1] the kk = 1 operands.
    bf16x8 af[2][C::FM], bfr[2][C::FN];
    auto read_frags = [&](int slot, int kk) {
      const char* sA = smem + slot * C::STAGE;
      const char* sB = sA + C::A_BYTES;
#pragma unroll
      for (int i = 0; i < C::FM; ++i) af[kk][i] = *reinterpret_cast<const bf16x8*>(sA + a_rd[kk] + i * 32 * 64);
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const bf16x4_t lo = lds_tr4(sB + b_rd[j] + kk * 16 * C::BROW);
        const bf16x4_t hi = lds_tr4(sB + b_rd[j] + kk * 16 * C::BROW + 4 * C::BROW);
        bfr[kk][j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    auto mfma = [&](int kk) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
        if (C::BM != 128 || i < fm_active) {  // the skip is for 128-row expert tiles only
#pragma unroll
          for (int j = 0; j < C::FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[kk][j], af[kk][i], acc[i][j], 0, 0, 0);
        }
    };

    if constexpr (C::WAVES == 8) {
      // Ping-pong schedule.  Waves 0-3 (group X) and 4-7 (group Y) hold one
      // wave of each SIMD.  Phases are separated by workgroup barriers; in
      // every phase one group runs a memory step M(j) (all LDS operand reads
      // of stage j into registers, plus the DMA of stage j+S-1 into the slot
      // stage j-1 left) while the other runs the compute step C (the stage's
      // MFMAs from registers), so each SIMD's MFMA pipe is fed by one wave
      // while its partner loads:
      //   phase 0:    X M(0)
      //   phase 2j+1: X C(j)    Y M(j)
      //   phase 2j+2: X M(j+1)  Y C(j)
      // Before the barrier that ends phase 2j+1 every wave waits for its own
      // DMA of stage j+1, so stage j+1 is complete when X reads it.
      const bool grp_x = wave_u < (uint32_t)(C::WAVES / 2);
      // Group X issues its DMA share before its operand reads, group Y after
      // them (Y's memory step shares its phase with both groups' DMA waits;
      // issuing after the reads measured 3 us faster on config 2 gated than
      // issuing first, and no slower elsewhere).  The DMA targets the slot
      // stage j-1 left, never the one being read.
      auto mem_step = [&](int j) {
        if (grp_x && j + C::S - 1 < nk) issue(j + C::S - 1);
        read_frags(j % C::S, 0);
        read_frags(j % C::S, 1);
        if (!grp_x && j + C::S - 1 < nk) issue(j + C::S - 1);
      };
      auto wait_j = [&](int j) { wait_stage<C::S + 1, C::LOADS>(min(C::S - 2, nk - 1 - j)); };
      // wait for stage j+1 (steady state: S-2 younger stages in flight)
      auto wait_next = [&](int j) {
        if (j + C::S - 1 < nk) wait_vm<(C::S - 2) * C::LOADS>();
        else if (j + 1 < nk) wait_j(j + 1);
      };
      auto bar = [] {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
      };
#pragma unroll
      for (int s = 0; s < C::S - 1; ++s)
        if (s < nk) issue(s);
      wait_j(0);
      __syncthreads();
      // The two groups run separate loops (same barrier count per iteration)
      // so each keeps a single set of fragment registers live.
      if (grp_x) {
        mem_step(0);
        for (int j = 0; j < nk; ++j) {
          bar();
          mfma(0);
          mfma(1);
          wait_next(j);
          bar();
          if (j + 1 < nk) mem_step(j + 1);
        }
      } else {
        for (int j = 0; j < nk; ++j) {
          bar();
          mem_step(j);
          wait_next(j);
          bar();
          mfma(0);
          mfma(1);
        }
      }
      // Every wave's last LDS read happened before the loop's final barrier,
      // so the ring is free for the next unit's prologue.
    } else {
      // Interleaved schedule (one wave per SIMD, S stages in flight).  Each
      // stage kt is two half-steps of NM MFMAs:
      //   A: MFMAs of sub-step 0 | reads of sub-step 1 (same stage)
      //   wait for stage kt+1, barrier
      //   B: MFMAs of sub-step 1 | refill of stage kt's slot with stage
      //      kt+S, then reads of stage kt+1 sub-step 0
      // and every LDS read and DMA instruction is pinned between two MFMAs:
      // one wave per SIMD has no partner wave to cover its issue slots, so
      // anything issued in a row with nothing in the matrix pipe is lost
      // MFMA time.  Issue is in order, so an instruction placed after an
      // MFMA goes out while that MFMA occupies the pipe.
      constexpr int NM = C::FM * C::FN;      // MFMAs per K sub-step
      constexpr int NR = C::FM + 2 * C::FN;  // LDS reads per K sub-step
      constexpr int NPA = C::A_INST / 2, NP = NPA + C::B_INST / 2;  // DMA pairs per stage
      static_assert(C::A_INST % 2 == 0 && C::B_INST % 2 == 0 && 2 * NP <= NM, "4-wave schedule shape");
      bf16x4_t blo[2][C::FN], bhi[2][C::FN];
      // read r of sub-step kk of ring slot `slot`: A fragments first, then
      // the two transposing halves of each B fragment
      auto rd = [&](int slot, int kk, int r) {
        const char* sA = smem + slot * C::STAGE;
        const char* sB = sA + C::A_BYTES;
        if (r < C::FM) {
          af[kk][r] = *reinterpret_cast<const bf16x8*>(sA + a_rd[kk] + r * 32 * 64);
        } else {
          const int j = (r - C::FM) >> 1;
          if (((r - C::FM) & 1) == 0) blo[kk][j] = lds_tr4(sB + b_rd[j] + kk * 16 * C::BROW);
          else bhi[kk][j] = lds_tr4(sB + b_rd[j] + kk * 16 * C::BROW + 4 * C::BROW);
        }
      };
      auto mm = [&](int kk, int x) {
        const int i = x / C::FN, j = x % C::FN;
        if (C::BM == 128 && i >= fm_active) return;  // padding-only 32-row block of an expert tile
        const bf16x8 bv = __builtin_shufflevector(blo[kk][j], bhi[kk][j], 0, 1, 2, 3, 4, 5, 6, 7);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bv, af[kk][i], acc[i][j], 0, 0, 0);
      };
      // NM MFMAs of sub-step kk starting at x0, with reads (rslot, rkk)
      // r = 0..NR-1 spread evenly behind them
      auto mfma_reads = [&](int kk, int x0, int rslot, int rkk) {
        constexpr int n = NM;  // upper bound of the loop below; x0 > 0 shortens it
#pragma unroll
        for (int x = 0; x < n; ++x) {
          if (x < x0) continue;
          mm(kk, x);
          const int r0 = (x - x0) * NR / (NM - x0), r1 = (x - x0 + 1) * NR / (NM - x0);
#pragma unroll
          for (int r = r0; r < r1; ++r) rd(rslot, rkk, r);
        }
#pragma unroll
        for (int x = 0; x < n; ++x) {
          if (x < x0) continue;
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          const int r0 = (x - x0) * NR / (NM - x0), r1 = (x - x0 + 1) * NR / (NM - x0);
#pragma unroll
          for (int r = r0; r < r1; ++r) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // its LDS reads
        }
        __builtin_amdgcn_sched_barrier(0);
      };
      // half-step B with the refill of slot kt % S by stage kt + S: the DMA
      // pairs ride behind the first 2*NP MFMAs (inline asm, pinned by
      // sched_barrier), the reads of stage kt+1 behind the rest
      auto half_b_refill = [&](int kt) {
        const uint32_t st = lds_base + (uint32_t)(kt % C::S) * C::STAGE;
        const uint32_t ka = (uint32_t)(k0 + kt + C::S) * (C::BKD * 2);
        const uint32_t kb = (uint32_t)(k0 + kt + C::S) * (C::BKD * p.ldb * 2);
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          mm(1, 2 * q);
          mm(1, 2 * q + 1);
          __builtin_amdgcn_sched_barrier(0);
          if (q < NPA) {
            const uint32_t l = st + wave_u * C::A_INST * 1024 + 2 * q * 1024;
            dma16x2(rA, l, l + 1024, a_src[2 * q], a_src[2 * q + 1], ka);
          } else {
            const int qb = q - NPA;
            const uint32_t l = st + C::A_BYTES + wave_u * C::B_INST * 1024 + 2 * qb * 1024;
            dma16x2(rB, l, l + 1024, b_src[2 * qb], b_src[2 * qb + 1], kb);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        mfma_reads(1, 2 * NP, (kt + 1) % C::S, 0);
      };
#pragma unroll
      for (int s = 0; s < C::S; ++s)
        if (s < nk) issue(s);
      wait_stage<C::S + 1, C::LOADS>(min(C::S - 1, nk - 1));
      __syncthreads();
#pragma unroll
      for (int r = 0; r < NR; ++r) rd(0, 0, r);
      int kt = 0;
      // steady state: every iteration refills the slot it finished
      for (; kt + C::S < nk; ++kt) {
        mfma_reads(0, 0, kt % C::S, 1);
        wait_vm<(C::S - 2) * C::LOADS>();  // stage kt+1 landed (S-2 younger stages in flight)
        __syncthreads();
        half_b_refill(kt);
      }
      // drain: every stage is issued
      for (; kt < nk - 1; ++kt) {
        mfma_reads(0, 0, kt % C::S, 1);
        wait_stage<C::S + 1, C::LOADS>(nk - 2 - kt);
        __syncthreads();
        mfma_reads(1, 0, (kt + 1) % C::S, 0);
      }
      mfma_reads(0, 0, (nk - 1) % C::S, 1);
#pragma unroll
      for (int x = 0; x < NM; ++x) mm(1, x);
      // Every wave must be done with the ring before the next unit's DMA.
      __syncthreads();
    }

    m0_out = m0;
    tn_out = tn;
  };

  // Whole tiles walk the (possibly arrival-permuted) order, skipping the
  // split set; the split set is the last tiles of the unpermuted order, so
  // which tiles are split, and hence every output bit, does not depend on
  // the arrival order.
  const int st_total = p.st_nblocks * kPieces;
  for (int w = 0; w < n_full_mine; ++w) {
    if (sp.claim) {
      claim_stage<C::NT>(p, need_pieces(p, sp, w), n_cons, reinterpret_cast<int*>(smem));
    } else if (sp.round_need && sp.gsize > 0 && w < sp.n_rounds) {
      alt_stage<C::NT>(p, cons_id, sp, w);
    } else if (sp.round_need) {
      // this tile is in round w: stage what round w waits for, and at least
      // an even share of the rest
      const int need = (sp.round_need[w] + 1) * kPieces;
      const int even = (int)((int64_t)st_total * (w + 1) / sp.n_rounds);
      coop_stage<C::NT>(p, n_cons, sp.q, sp.batch, max(need, even));
    }
    int t = (w < last_round ? cons_id : last_slot) + w * n_cons;
    if (full_list) t = full_list[t];
    f32x16 acc[C::FM][C::FN];
    int m0, tn;
    tile_body(t, row_perm != nullptr, 0, nk_all, acc, m0, tn);
    store_tile<C, EPI>(p, acc, m0, tn, tid, smem);
  }
  if (sp.round_need && !sp.claim && sp.gsize == 0) coop_stage<C::NT>(p, n_cons, sp.q, sp.batch, st_total);
  // claimed mode: the K-split tail tiles may wait for pieces past every
  // whole round's need; claim whatever is still unclaimed (normally nothing:
  // the staging kernel is ahead), so no piece is left to a kernel that might
  // not be running
  if (sp.claim) {
    claim_stage<C::NT>(p, st_total, n_cons, reinterpret_cast<int*>(smem));
    if (tid == 0) claim_checkout(p, p.st_claimers + p.st_stage_waves);
  }
  // alternating mode: a consumer with no tile in the last whole round
  // still copies its shares of the ranges staged before that round
  if (sp.round_need && sp.gsize > 0)
    for (int w = n_full_mine; w < sp.n_rounds; ++w) alt_stage<C::NT>(p, cons_id, sp, w);
  if (cons_id >= n_tail_units) return;
  // The K-split unit: tail tile full + tail_idx (unpermuted), K part `part`.
  const int tail_idx = cons_id / sk_split;
  const int part = cons_id % sk_split;
  const int k0 = part * nk_all / sk_split;
  const int nk = (part + 1) * nk_all / sk_split - k0;
  f32x16 acc[C::FM][C::FN];
  int m0, tn;
  tile_body(full + tail_idx, false, k0, nk, acc, m0, tn);
  if (C::WM == 2 && sk_split == 2 && EPI != kEpiReduce) {
    // Two-way split: the parts swap half tiles.  Part q finalizes the rows
    // of the waves with wm == q (rows q*WTM .. q*WTM + WTM - 1): the other
    // waves write their fp32 partial to this part's slot, and after the
    // other part's flag the owning waves add its partial and store their
    // rows.  Both workgroups of the tile finish together, each moving half
    // of the tile (one owner folding the whole tile measured ~33 us while
    // the contributor sat idle).  Each element is the sum of the same two
    // fp32 terms as with one owner (a two-term sum does not depend on order).
    const int slot_out = tail_idx * 2 + part, slot_in = tail_idx * 2 + (1 - part);
    const bool own_rows = wm == part;
    if (!own_rows) put_partial<C>(p.sk_ws + (int64_t)slot_out * (C::BM * C::BN), acc, tid);
    // write-through stores performed at agent scope, then a relaxed flag
    // (the protocol of copy_wt: no L2 write-back needed)
    wait_vmem_all();
    __syncthreads();
    if (tid == 0) {
      __hip_atomic_store(p.sk_flags + slot_out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_flags<1>([&](int) { return p.sk_flags + slot_in; }, 1, 1u, p.spin_limit, p.err);
    }
    __syncthreads();
    if (own_rows) {
      // two fp32 terms: the sum is the same whichever part adds
      add_partial_regs<C>(p.sk_ws + (int64_t)slot_in * (C::BM * C::BN), acc, tid);
      store_tile<C, EPI>(p, acc, m0, tn, tid, smem);
    }
    __syncthreads();  // the partial is read: clear its flag for the next launch
    if (tid == 0) __hip_atomic_store(p.sk_flags + slot_in, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (part > 0) {
    // K-split contributor: publish the partial for part 0 of this tile.
    const int slot = tail_idx * (sk_split - 1) + part - 1;
    put_partial<C>(p.sk_ws + (int64_t)slot * (C::BM * C::BN), acc, tid);
    // write-through stores performed at agent scope, then a relaxed flag
    // (the protocol of copy_wt: no L2 write-back needed)
    wait_vmem_all();
    __syncthreads();
    if (tid == 0) __hip_atomic_store(p.sk_flags + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  {
    // K-split owner: acquire every contributor's partial, fold in part
    // order, and clear the flags for the next launch on this workspace.
    const int slot0 = tail_idx * (sk_split - 1);
    if (tid == 0)
      // one flag at a time: the split unit's registers are at the limit
      for (int q2 = 0; q2 < sk_split - 1; ++q2)
        wait_flags<1>([&](int) { return p.sk_flags + slot0 + q2; }, 1, 1u, p.spin_limit, p.err);
    __syncthreads();
    for (int q2 = 0; q2 < sk_split - 1; ++q2)
      add_partial<C>(p.sk_ws + (int64_t)(slot0 + q2) * (C::BM * C::BN), acc, tid, smem);
    if (tid == 0)
      for (int q2 = 0; q2 < sk_split - 1; ++q2)
        __hip_atomic_store(p.sk_flags + slot0 + q2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  store_tile<C, EPI>(p, acc, m0, tn, tid, smem);
}

// Order of row tiles for a gated consumer: ascending by the stage position at
// which the last 128-row flag of the tile is published (ties by row), so
// compute follows arrival; for the reduce epilogue, the owned rows spread one
// per round among the others.
template <int BM, int NT>
__device__ void build_row_perm(const GemmKParams& p, int* row_perm, int* row_key, int* scratch) {
  const int tid = threadIdx.x;
  const int tm = p.tiles_m;
  if (p.perm_mode == kPermArrival || p.perm_mode == kPermPeerArrival) {
    // Row tile i waits for flags: its own BM/128 flags (AllGather), or those
    // of every peer for its rows (all-reduce: flag q * rbs + row block).
    const int per = BM / kFlagRows;
    const int npeer = p.perm_mode == kPermPeerArrival ? p.rs_npeers : 1;
    const int rbs = tm * per;  // flags per peer
    const int nflag = npeer * rbs;
    for (int i = tid; i < nflag; i += NT) {
      const int f = p.a_stage_order[i];
      if ((unsigned)f < (unsigned)nflag) scratch[f] = i;  // flag -> position
    }
    __syncthreads();
    for (int i = tid; i < tm; i += NT) {
      int key = 0;
      for (int q = 0; q < npeer; ++q)
        for (int f = 0; f < per; ++f) key = max(key, scratch[q * rbs + i * per + f]);
      scratch[nflag + i] = key;
    }
    __syncthreads();
    for (int i = tid; i < tm; i += NT) {
      const int key = scratch[nflag + i];
      int rank = 0;
      for (int j = 0; j < tm; ++j) {
        const int kj = scratch[nflag + j];
        rank += (kj < key) || (kj == key && j < i);
      }
      row_perm[rank] = i;
      row_key[rank] = key;
    }
  } else if (p.perm_mode == kPermOwnedSpread) {
    // Owned row tiles spread over the order: the owned row of arrival rank k
    // sits in segment k of nown equal segments, at offset k % L (L = the
    // segment length), so with one segment per round every round folds one
    // owned row and the folding workgroups rotate from round to round
    // (reference: the device-relative slice interleave of
    // include/operators/gemm_rs/gemm_rs.cuh:306-318).  An owned row's
    // arrival key is the last stage position among its peers' blocks when
    // this launch stages them (so a row-block-major stage order lets round
    // k fold the k-th row), else its index.
    const int own0 = p.rs_own_row0 / BM, nown = p.rs_own_rows / BM;
    const int per = BM / kFlagRows, rbs = p.rs_own_rows / kFlagRows;
    const bool staged = p.st_nblocks > 0 && (p.st_coop || p.n_prod > 0);
    int* pos = scratch;                        // flag -> stage position
    int* okey = scratch + p.st_nblocks;        // owned row -> arrival key
    int* oby = okey + nown;                    // arrival rank -> owned row
    if (staged) {
      for (int i = tid; i < p.st_nblocks; i += NT) {
        const int f = p.st_order ? p.st_order[i] : i;
        if ((unsigned)f < (unsigned)p.st_nblocks) pos[f] = i;
      }
    }
    __syncthreads();
    for (int k = tid; k < nown; k += NT) {
      int key = k;
      if (staged) {
        key = 0;
        for (int q = 0; q < p.rs_npeers; ++q)
          for (int sub = 0; sub < per; ++sub) key = max(key, pos[q * rbs + k * per + sub]);
      }
      okey[k] = key;
    }
    __syncthreads();
    for (int k = tid; k < nown; k += NT) {
      int rank = 0;
      for (int j = 0; j < nown; ++j) rank += (okey[j] < okey[k]) || (okey[j] == okey[k] && j < k);
      oby[rank] = k;
    }
    __syncthreads();
    const int L = max(tm / max(nown, 1), 1);
    auto seg_start = [&](int k) { return (int)((int64_t)k * tm / nown); };
    for (int i = tid; i < tm; i += NT) {
      int r, key = -1;
      if (nown == 0) {
        r = i;
      } else {
        int k = (int)((int64_t)i * nown / tm);
        while (k + 1 < nown && seg_start(k + 1) <= i) ++k;
        while (k > 0 && seg_start(k) > i) --k;
        const int slot = seg_start(k) + k % L;
        if (i == slot) {
          r = own0 + oby[k];
          key = staged ? okey[oby[k]] : -1;
        } else {
          const int j = i - k - (i > slot ? 1 : 0);  // index among the non-owned rows
          r = j < own0 ? j : j + nown;
        }
      }
      row_perm[i] = r;
      row_key[i] = key;
    }
  }
  __syncthreads();
}

// Staging need of each whole-tile round: round_need[r] = the last stage
// position any tile of round r (whole tiles i = r*n_cons .. (r+1)*n_cons-1
// of the schedule) waits for.  Staging every piece up to that position
// before round r, in every workgroup, lets round r complete without waiting
// on a workgroup that is still in an earlier round.
template <int NT>
__device__ void build_round_need(const GemmKParams& p, int full, int n_rounds, const uint16_t* full_list,
                                 const int* row_key, int* round_need) {
  const int tid = threadIdx.x;
  for (int r = tid; r < n_rounds; r += NT) round_need[r] = -1;
  __syncthreads();
  for (int i = tid; i < full; i += NT) {
    const int t = full_list ? full_list[i] : i;
    int tm, tn;
    decode_grouped(t, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    atomicMax(&round_need[i / p.n_cons], row_key[tm]);
  }
  __syncthreads();
}

// Unpermuted tile index of tile (tm, tn): the inverse of decode_grouped.
__device__ __forceinline__ int encode_grouped(int tm, int tn, int tiles_m, int tiles_n, int group_m) {
  const int g = tm / group_m;
  const int first = g * group_m;
  const int gm = min(tiles_m - first, group_m);
  return g * group_m * tiles_n + tn * gm + (tm - first);
}

// Positions of the arrival-permuted order whose tile is not in the split set
// (tiles sk_full.. of the unpermuted order), in order: full_list[i] is the
// position of the i-th whole tile.  Each thread takes a contiguous chunk of
// positions; a block-wide scan of the chunk counts gives the output offsets.
template <int NT>
__device__ void build_full_list(const GemmKParams& p, const int* row_perm, uint16_t* full_list, int* scratch) {
  const int tid = threadIdx.x;
  const int ntiles = p.tiles_m * p.tiles_n;
  const int per = (ntiles + NT - 1) / NT;
  const int lo = min(tid * per, ntiles), hi = min(lo + per, ntiles);
  auto whole = [&](int pos) {
    int tm, tn;
    decode_grouped(pos, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    return encode_grouped(row_perm[tm], tn, p.tiles_m, p.tiles_n, p.group_m) < p.sk_full;
  };
  int c = 0;
  for (int i = lo; i < hi; ++i) c += whole(i);
  scratch[tid] = c;
  __syncthreads();
  for (int off = 1; off < NT; off <<= 1) {
    const int v = tid >= off ? scratch[tid - off] : 0;
    __syncthreads();
    scratch[tid] += v;
    __syncthreads();
  }
  int o = scratch[tid] - c;
  for (int i = lo; i < hi; ++i)
    if (whole(i)) full_list[o++] = (uint16_t)i;
  __syncthreads();
}

template <int BM, int WAVES, int EPI, int BN>
__device__ __forceinline__ void gemm_main(const GemmKParams& p) {
  using C = Cfg<BM, WAVES, BN>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  if ((int)blockIdx.x < p.n_prod) {
    producer_role<C::NT>(p, blockIdx.x);
    return;
  }
  int cons = blockIdx.x - p.n_prod;
  int n_cons = p.n_cons;
  if constexpr (BM == 128) {
    // Device row count with the library's grid: when the tail round cannot
    // be K-split (more tail tiles than half the grid), every consumer runs
    // the same number of whole-tile rounds anyway, so spread the tiles over
    // the fewest consumers (a multiple of 8) that keep that round count —
    // the host's rule for host-sized launches; the others exit here.
    if (p.rows_dev && p.spread_dev) {
      const int64_t rows = *p.rows_dev;
      const int nt = (int)min<int64_t>(p.tiles_m, max<int64_t>(rows, 0) / C::BM) * p.tiles_n;
      const int R = nt % n_cons;
      if (R != 0 && 2 * R > n_cons) {
        const int rounds = (nt + n_cons - 1) / n_cons;
        const int even = ((nt + rounds - 1) / rounds + 7) / 8 * 8;
        if (even < n_cons) {
          if (cons >= even) return;
          n_cons = even;
        }
      }
      n_cons = __builtin_amdgcn_readfirstlane(n_cons);
    }
  }
  // XCD-aware renumbering: workgroups are dealt round-robin to the 8 XCDs,
  // so give each XCD a contiguous run of consumer ids (hence of tiles, which
  // the grouped order keeps close in A rows / B columns) for L2 reuse.
  if (p.xcd_remap) cons = (cons % 8) * (n_cons / 8) + cons / 8;
  StagePlan sp;
  sp.q = cons;
  sp.batch = 1;
  sp.n_rounds = 0;
  sp.round_need = nullptr;
  sp.grp = sp.gid = sp.gsize = 0;
  sp.claim = false;
  if constexpr (C::kSched) {
    __shared__ int row_perm[kMaxTilesM];
    __shared__ uint16_t full_list[kMaxSplitListTiles];
    __shared__ int row_key[kMaxTilesM];
    __shared__ int round_need[kMaxRounds];
    const int* perm = nullptr;
    if (p.perm_mode != kPermNone) {
      build_row_perm<BM, C::NT>(p, row_perm, row_key, reinterpret_cast<int*>(smem));
      perm = row_perm;
    }
    const uint16_t* flist = nullptr;
    if (perm && p.sk_split > 1) {
      build_full_list<C::NT>(p, row_perm, full_list, reinterpret_cast<int*>(smem));
      flist = full_list;
    }
    // Cooperative staging runs between tile rounds when the schedule's
    // staging needs are known (a permuted order with at most kMaxRounds
    // rounds); otherwise all of it runs before the first tile.
    if (p.st_coop) {
      const int ntiles = p.tiles_m * p.tiles_n;
      const int full = (p.sk_split > 1) ? p.sk_full : ntiles;
      const int n_rounds = (full + p.n_cons - 1) / p.n_cons;
      if (perm && n_rounds <= kMaxRounds) {
        build_round_need<C::NT>(p, full, n_rounds, flist, row_key, round_need);
        sp.n_rounds = n_rounds;
        sp.round_need = round_need;
        sp.claim = p.st_coop == 3;
        if (p.st_coop == 2 && p.xcd_remap && n_rounds >= 1) {
          sp.gsize = p.n_cons / 2;
          sp.grp = cons / sp.gsize;
          sp.gid = cons % sp.gsize;
        }
      } else if (p.st_coop == 3) {
        // no per-round needs known: claim an even share of everything now
        claim_stage<C::NT>(p, p.st_nblocks * kPieces, p.n_cons, reinterpret_cast<int*>(smem));
        if (threadIdx.x == 0) claim_checkout(p, p.st_claimers + p.st_stage_waves);
      } else {
        coop_stage<C::NT>(p, p.n_cons, sp.q, sp.batch, p.st_nblocks * kPieces);
      }
    }
    compute_role<C, EPI>(p, cons, p.n_cons, smem, perm, flist, sp);
  } else {
    // 128-row kernels: no arrival order and no staging (the host never
    // launches them with either); cooperative staging, if asked for, runs
    // before the first tile.
    if (p.st_coop) coop_stage<C::NT>(p, p.n_cons, sp.q, sp.batch, p.st_nblocks * kPieces);
    compute_role<C, EPI>(p, cons, n_cons, smem, nullptr, nullptr, sp);
  }
}

template <int BM, int WAVES, int EPI, int BN>
__global__ __launch_bounds__(64 * WAVES, 1) void gemm_kernel(GemmKParams p) {
  gemm_main<BM, WAVES, EPI, BN>(p);
}

// The 256 x 256 GEMM that runs beside the staging kernel, capped at 224
// VGPRs per wave (the attribute counts in units of two registers on gfx950,
// whose waves draw VGPRs and AGPRs from one 512-entry file per SIMD lane):
// its two waves per SIMD leave 64 registers on every SIMD for one staging
// wave.  The K loop stays spill-free at this cap (the extra spills are in
// the tile set-up and the K-split exchange).
template <int EPI>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_num_vgpr(112))) void gemm_kernel_capped(GemmKParams p) {
  gemm_main<256, 8, EPI, 256>(p);
}

// One thread: *epoch_ptr + 1, skipping 0 (a vector store, ordered before
// the next launch on the stream by the kernel boundary).
__global__ void epoch_advance_kernel(uint32_t* epoch_ptr) {
  if (threadIdx.x == 0) {
    uint32_t e = __hip_atomic_load(epoch_ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (e == 0u) e = 1u;
    __hip_atomic_store(epoch_ptr, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

hipError_t launch_epoch_advance(uint32_t* epoch_ptr, hipStream_t stream) {
  hipLaunchKernelGGL(epoch_advance_kernel, dim3(1), dim3(64), 0, stream, epoch_ptr);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int BM, int WAVES, int EPI, int BN>
static hipError_t launch_t(const GemmKParams& p, hipStream_t stream) {
  using C = Cfg<BM, WAVES, BN>;
  // The dynamic-LDS limit is raised once per device and kernel.  Two
  // threads that both find the flag clear both set the attribute, which is
  // harmless; a launch never runs before its device's attribute is set.
  static PerDeviceFlag attr_set;
  constexpr uint32_t lds = C::LDS_BYTES;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (!attr_set.is_set(dev)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, WAVES, EPI, BN>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_set.set(dev);
  }
  hipLaunchKernelGGL((gemm_kernel<BM, WAVES, EPI, BN>), dim3(p.n_prod + p.n_cons), dim3(C::NT), lds, stream, p);
  return hipGetLastError();
}

template <int BM, int EPI>
static hipError_t launch_w(const GemmKParams& p, hipStream_t stream) {
  return p.waves == 8 ? launch_t<BM, 8, EPI, 256>(p, stream) : launch_t<BM, 4, EPI, 256>(p, stream);
}

// Side stream and fork/join events of the co-resident staging, one set per
// device, created on first use and kept until the process ends.
struct CostageStreams {
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

static hipError_t costage_streams(int dev, CostageStreams** out) {
  static std::mutex mu;
  static std::vector<CostageStreams> per_dev;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)per_dev.size() <= dev) per_dev.resize(dev + 1);
  CostageStreams& c = per_dev[dev];
  if (!c.side) {
    hipError_t e = hipStreamCreateWithFlags(&c.side, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c.fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c.join, hipEventDisableTiming);
    if (e != hipSuccess) return e;
  }
  *out = &c;
  return hipSuccess;
}

hipError_t launch_gemm_costaged(const GemmKParams& p, int epi, int n_stage_waves, hipStream_t stream) {
  using C = Cfg<256, 8, 256>;
  if (p.waves != 8 || p.st_coop != 3 || !p.st_claim || n_stage_waves < 1) return hipErrorInvalidValue;
  if (epi != kEpiStore && epi != kEpiReduce) return hipErrorInvalidValue;
  const void* fn = epi == kEpiReduce ? reinterpret_cast<const void*>(&gemm_kernel_capped<kEpiReduce>)
                                     : reinterpret_cast<const void*>(&gemm_kernel_capped<kEpiStore>);
  static PerDeviceFlag attr_set[2];
  PerDeviceFlag& flag = attr_set[epi == kEpiReduce ? 1 : 0];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint32_t lds = C::LDS_BYTES;
  if (!flag.is_set(dev)) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    flag.set(dev);
  }
  CostageStreams* cs = nullptr;
  if ((e = costage_streams(dev, &cs)) != hipSuccess) return e;
  // Fork: the staging kernel is enqueued first, on the side stream, after
  // everything already on `stream`; the GEMM follows on `stream`; the join
  // makes later work on `stream` wait for both.  The two kernels run
  // concurrently when the streams sit on different hardware queues (the
  // GEMM's register cap leaves room for the staging waves on every SIMD);
  // on one queue they run one after the other, staging first.  Either way
  // nothing waits in a cycle: the staging waves wait on nothing.
  GemmKParams pg = p;
  // claimers that check out of the claim word: every compute workgroup and
  // every staging wave
  pg.st_claimers = p.n_cons;
  pg.st_stage_waves = n_stage_waves;
  if ((e = hipEventRecord(cs->fork, stream)) != hipSuccess) return e;
  if ((e = hipStreamWaitEvent(cs->side, cs->fork, 0)) != hipSuccess) return e;
  hipLaunchKernelGGL(stage_kernel, dim3(n_stage_waves), dim3(64), 0, cs->side, pg);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = hipEventRecord(cs->join, cs->side)) != hipSuccess) return e;
  GemmKParams pk = pg;
  void* args[] = {&pk};
  if ((e = hipLaunchKernel(fn, dim3(p.n_prod + p.n_cons), dim3(C::NT), args, lds, stream)) != hipSuccess)
    return e;
  return hipStreamWaitEvent(stream, cs->join, 0);
}

// Tile BM x bn; bn = 512 exists for BM = 128 with the store and SwiGLU
// epilogues (the grouped expert GEMMs: half the activation re-streaming per
// weight byte of the 128 x 256 tile) and 8 waves.
hipError_t launch_gemm(const GemmKParams& p, int bm, int epi, hipStream_t stream, int bn) {
  if (bn == 512) {
    if (bm != 128 || p.waves != 8) return hipErrorInvalidValue;
    if (epi == kEpiStore) return launch_t<128, 8, kEpiStore, 512>(p, stream);
    if (epi == kEpiSwiGLU) return launch_t<128, 8, kEpiSwiGLU, 512>(p, stream);
    return hipErrorInvalidValue;
  }
  if (bn != 256) return hipErrorInvalidValue;
  if (bm == 256) {
    if (epi == kEpiStore) return launch_w<256, kEpiStore>(p, stream);
    if (epi == kEpiReduce) return launch_w<256, kEpiReduce>(p, stream);
    if (epi == kEpiSwiGLU) return launch_w<256, kEpiSwiGLU>(p, stream);
  } else if (bm == 128) {
    if (epi == kEpiStore) return launch_w<128, kEpiStore>(p, stream);
    if (epi == kEpiReduce) return launch_w<128, kEpiReduce>(p, stream);
    if (epi == kEpiSwiGLU) return launch_w<128, kEpiSwiGLU>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mk
