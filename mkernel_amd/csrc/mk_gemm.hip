// mk_gemm.hip — persistent, tile-scheduled bf16 GEMM for gfx950 with
// workgroup roles:
//   * producer workgroups (blockIdx.x < n_prod) stage 128-row tiles of HBM
//     data (AllGather shards or peer partials) and release-store a flag per
//     tile — the in-GPU stand-in for the reference's intra_comm_sm gather
//     (reference src/ag_gemm.cu:31-215);
//   * compute workgroups run BMx256x64 tiles on v_mfma_f32_32x32x16_bf16 with
//     a double-buffered LDS pipeline, optionally acquire-waiting the A-row
//     flags before a tile (reference src/ag_gemm.cu:374-377) and optionally
//     folding staged peer partials into the epilogue (reference
//     src/gemm_rs.cu:685-845 reduce_tiles_ws, here in fp32 with one rounding).
//
// Operand layout: A row-major [M,K]; B row-major [K,N] (as the reference
// stores weights, bench/dispatch_gemm_glu_combine_bench.py:546-553).  B is
// transposed on its way into LDS (8x8 register transpose with v_perm_b32), so
// both LDS tiles are K-contiguous and every MFMA operand read is one
// ds_read_b128.  The MFMA is issued as (B-fragment, A-fragment) so that each
// lane's accumulator holds 4 consecutive N values of one row: the epilogue
// writes 8-byte row segments.
#include "mk_device.h"
#include "mk_internal.h"

namespace mk {

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

// ---------------------------------------------------------------------------
// Producer role: copy 128-row blocks src -> dst in stage order, then publish.
// ---------------------------------------------------------------------------
__device__ void producer_role(const GemmKParams& p, int pid) {
  const int64_t block_elems = (int64_t)kFlagRows * p.st_cols;
  const int64_t block_vec = block_elems / 8;  // uint4 units
  constexpr int U = 8;
  for (int i = pid; i < p.st_nblocks; i += p.n_prod) {
    const int b = p.st_order ? p.st_order[i] : i;
    const uint4* src = reinterpret_cast<const uint4*>(p.st_src + (int64_t)b * block_elems);
    uint4* dst = reinterpret_cast<uint4*>(p.st_dst + (int64_t)b * block_elems);
    int64_t base = threadIdx.x;
    for (; base + (int64_t)(U - 1) * kThreads < block_vec; base += (int64_t)U * kThreads) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = src[base + u * kThreads];
#pragma unroll
      for (int u = 0; u < U; ++u) dst[base + u * kThreads] = v[u];
    }
    for (; base < block_vec; base += kThreads) dst[base] = src[base];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) publish_flag(p.st_flags + b, p.epoch);
  }
}

// ---------------------------------------------------------------------------
// Compute role
// ---------------------------------------------------------------------------
template <int BM>
struct TileCfg {
  static constexpr int WM = 2, WN = 2;
  static constexpr int WTM = BM / WM;     // wave tile rows
  static constexpr int WTN = kBN / WN;    // wave tile cols (128)
  static constexpr int FM = WTM / 32;     // 32x32 blocks per wave (M)
  static constexpr int FN = WTN / 32;     // (N) = 4
  static constexpr int A_LD = BM / 32;    // uint4 A loads per thread per stage
  static constexpr uint32_t A_BYTES = BM * 128;
  static constexpr uint32_t B_BYTES = kBN * 128;
  static constexpr uint32_t STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr uint32_t LDS_BYTES = 2 * STAGE_BYTES;
};

// Global column of B for LDS B-row q (q multiple of 8 — one 16-byte chunk).
template <int EPI>
__device__ __forceinline__ int b_col(const GemmKParams& p, int tn, int q) {
  if constexpr (EPI == kEpiSwiGLU) {
    constexpr int WTN = kBN / 2;
    constexpr int half = WTN / 2;
    const int wn = q / WTN, r = q % WTN;
    const int base = tn * (kBN / 2) + wn * half;
    return r < half ? base + r : p.swiglu_I + base + (r - half);
  } else {
    return tn * kBN + q;
  }
}

template <int BM, int EPI>
__device__ void compute_role(const GemmKParams& p, int cons_id, char* smem, int* row_perm) {
  using C = TileCfg<BM>;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / C::WN;
  const int wn = wave % C::WN;
  const int ml = lane & 31;   // row inside a 32x32 block (M side)
  const int kg = lane >> 5;   // which 8-wide K half of the 16-wide MFMA step

  const int ntiles = p.tiles_m * p.tiles_n;
  const int nk = p.K / kBK;

  // B staging: one 8(k) x 8(n) block per thread per stage.  Within each
  // 16-lane group, lanes span 4 column chunks x 4 k-groups (so the
  // transposed LDS stores are conflict-free) and 16 consecutive chunks of one
  // k-row (so each global load reads 256 contiguous bytes per k-row).
  const int b_nc = (lane & 3) | ((lane >> 4) << 2) | ((wave & 1) << 4);  // 0..31
  const int b_kg = ((lane >> 2) & 3) | ((wave >> 1) << 2);              // 0..7

  // Per-thread LDS offsets.  Rows 32 apart share the swizzle, so one offset
  // per K sub-step serves every 32x32 block of the wave.
  const uint32_t a_st_off = lds_off(tid >> 3, tid & 7);
  uint32_t rd_off[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) rd_off[kk] = lds_off(ml, 2 * kk + kg);

  for (int t = cons_id; t < ntiles; t += p.n_cons) {
    int tm, tn;
    decode_grouped(t, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    if (row_perm) tm = row_perm[tm];
    // Tile coordinates are wave-uniform; keep them in SGPRs so the buffer
    // resources below stay scalar.
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    const int m0 = tm * BM;

    const uint16_t* Bp = p.B;
    if (p.rb_expert) {
      const int e = __builtin_amdgcn_readfirstlane(p.rb_expert[tm]);
      Bp += (int64_t)e * p.b_expert_stride;
    } else if (p.expert_rows) {
      // Expert whose padded row range holds row m0 (prefix walk over the
      // per-expert padded counts; E is small).
      int e = 0, end = 0;
      for (; e < p.n_experts; ++e) {
        end += p.expert_rows[e];
        if (tm * BM < end) break;
      }
      e = __builtin_amdgcn_readfirstlane(min(e, p.n_experts - 1));
      Bp += (int64_t)e * p.b_expert_stride;
    }

    // --- flag gate on the A rows of this tile (AllGather consumer side) ---
    if (p.a_flags) {
      if (tid < BM / kFlagRows) wait_flag(p.a_flags + (m0 / kFlagRows) + tid, p.epoch, p.spin_limit, p.err);
      __syncthreads();
    }

    // Buffer resources over this tile's A rows and this expert's B.
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)(BM * p.lda * 2));
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(Bp, (uint32_t)(p.K * p.ldb * 2));
    const uint32_t a_voff = (uint32_t)((tid >> 3) * p.lda * 2 + (tid & 7) * 16);
    const uint32_t a_row32 = (uint32_t)(32 * p.lda * 2);
    const uint32_t b_voff = (uint32_t)((b_kg * 8) * p.ldb * 2 + b_col<EPI>(p, tn, b_nc * 8) * 2);
    const uint32_t b_row = (uint32_t)(p.ldb * 2);

    uint4 ra[C::A_LD];
    uint4 rb[8];

    auto load_stage = [&](int kt) {
      const uint32_t ka = (uint32_t)kt * (kBK * 2);
#pragma unroll
      for (int i = 0; i < C::A_LD; ++i) ra[i] = buf_load16(rA, a_voff, ka + i * a_row32);
      const uint32_t kb = (uint32_t)kt * kBK * b_row;
#pragma unroll
      for (int j = 0; j < 8; ++j) rb[j] = buf_load16(rB, b_voff, kb + j * b_row);
    };
    auto store_stage = [&](int buf) {
      char* sA = smem + buf * C::STAGE_BYTES;
      char* sB = sA + C::A_BYTES;
#pragma unroll
      for (int i = 0; i < C::A_LD; ++i) *reinterpret_cast<uint4*>(sA + a_st_off + i * 4096) = ra[i];
      // 8x8 transpose: rb[j] holds B[k=8*b_kg+j][n=8*b_nc .. +7]; LDS row n
      // needs k = 8*b_kg .. +7 contiguous.
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
        const int d = i >> 1;
        uint4 o;
        o.x = __builtin_amdgcn_perm(((const uint32_t*)&rb[1])[d], ((const uint32_t*)&rb[0])[d], sel);
        o.y = __builtin_amdgcn_perm(((const uint32_t*)&rb[3])[d], ((const uint32_t*)&rb[2])[d], sel);
        o.z = __builtin_amdgcn_perm(((const uint32_t*)&rb[5])[d], ((const uint32_t*)&rb[4])[d], sel);
        o.w = __builtin_amdgcn_perm(((const uint32_t*)&rb[7])[d], ((const uint32_t*)&rb[6])[d], sel);
        *reinterpret_cast<uint4*>(sB + lds_off(b_nc * 8 + i, b_kg)) = o;
      }
    };

    f32x16 acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    load_stage(0);
    store_stage(0);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_stage(kt + 1);
      const char* sA = smem + cur * C::STAGE_BYTES + wm * C::WTM * 128;
      const char* sB = smem + cur * C::STAGE_BYTES + C::A_BYTES + wn * C::WTN * 128;
#pragma unroll
      for (int kk = 0; kk < kBK / 16; ++kk) {
        bf16x8 af[C::FM], bfr[C::FN];
#pragma unroll
        for (int i = 0; i < C::FM; ++i) af[i] = *reinterpret_cast<const bf16x8*>(sA + rd_off[kk] + i * 4096);
#pragma unroll
        for (int j = 0; j < C::FN; ++j) bfr[j] = *reinterpret_cast<const bf16x8*>(sB + rd_off[kk] + j * 4096);
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
          for (int j = 0; j < C::FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < nk) store_stage(cur ^ 1);
      __syncthreads();
    }

    // --- epilogue ---------------------------------------------------------
    // acc[i][j][4a+b] is C[m][n] with m = m0 + wm*WTM + 32i + ml and
    // n (in tile) = wn*WTN + 32j + 8a + 4kg + b.
    if constexpr (EPI == kEpiStore) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const int m = m0 + wm * C::WTM + i * 32 + ml;
        uint16_t* crow = p.C + (int64_t)m * p.ldc + tn * kBN + wn * C::WTN + 4 * kg;
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            uint2 w;
            w.x = pack_bf16x2(acc[i][j][4 * a + 0], acc[i][j][4 * a + 1]);
            w.y = pack_bf16x2(acc[i][j][4 * a + 2], acc[i][j][4 * a + 3]);
            *reinterpret_cast<uint2*>(crow + j * 32 + 8 * a) = w;
          }
      }
    } else if constexpr (EPI == kEpiSwiGLU) {
      // silu(g) * u in fp32, g = x / (1 + e^-x) as the reference computes it
      // (reference src/dispatch_gemm_glu_combine.cu:616-633).
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const int m = m0 + wm * C::WTM + i * 32 + ml;
        uint16_t* crow = p.C + (int64_t)m * p.ldc + tn * (kBN / 2) + wn * (C::WTN / 2) + 4 * kg;
#pragma unroll
        for (int j = 0; j < C::FN / 2; ++j)
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            float o[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              const float g = acc[i][j][4 * a + b];
              const float u = acc[i][j + C::FN / 2][4 * a + b];
              o[b] = (g / (1.0f + __expf(-g))) * u;
            }
            uint2 w;
            w.x = pack_bf16x2(o[0], o[1]);
            w.y = pack_bf16x2(o[2], o[3]);
            *reinterpret_cast<uint2*>(crow + j * 32 + 8 * a) = w;
          }
      }
    } else {  // kEpiReduce
      const bool owned = m0 >= p.rs_own_row0 && m0 < p.rs_own_row0 + p.rs_own_rows;
      if (!owned) {
#pragma unroll
        for (int i = 0; i < C::FM; ++i) {
          const int m = m0 + wm * C::WTM + i * 32 + ml;
          uint16_t* crow = p.C + (int64_t)m * p.ldc + tn * kBN + wn * C::WTN + 4 * kg;
#pragma unroll
          for (int j = 0; j < C::FN; ++j)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
              uint2 w;
              w.x = pack_bf16x2(acc[i][j][4 * a + 0], acc[i][j][4 * a + 1]);
              w.y = pack_bf16x2(acc[i][j][4 * a + 2], acc[i][j][4 * a + 3]);
              *reinterpret_cast<uint2*>(crow + j * 32 + 8 * a) = w;
            }
        }
      } else {
        const int lr0 = m0 - p.rs_own_row0;  // row inside the owned slice
        if (p.rs_flags) {
          const int rbs = p.rs_own_rows / kFlagRows;
          const int nf = p.rs_npeers * (BM / kFlagRows);
          if (tid < nf) {
            const int peer = tid / (BM / kFlagRows);
            const int rb = lr0 / kFlagRows + tid % (BM / kFlagRows);
            wait_flag(p.rs_flags + peer * rbs + rb, p.epoch, p.spin_limit, p.err);
          }
          __syncthreads();
        }
        const int64_t peer_stride = (int64_t)p.rs_own_rows * p.ldc;
#pragma unroll
        for (int i = 0; i < C::FM; ++i) {
          const int lr = lr0 + wm * C::WTM + i * 32 + ml;
          const int64_t off = (int64_t)lr * p.ldc + tn * kBN + wn * C::WTN + 4 * kg;
#pragma unroll
          for (int j = 0; j < C::FN; ++j)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
              float s0 = acc[i][j][4 * a + 0], s1 = acc[i][j][4 * a + 1];
              float s2 = acc[i][j][4 * a + 2], s3 = acc[i][j][4 * a + 3];
              for (int q = 0; q < p.rs_npeers; ++q) {
                const uint2 w = *reinterpret_cast<const uint2*>(p.rs_recv + q * peer_stride + off + j * 32 + 8 * a);
                s0 += bf16_lo(w.x);
                s1 += bf16_hi(w.x);
                s2 += bf16_lo(w.y);
                s3 += bf16_hi(w.y);
              }
              uint2 w;
              w.x = pack_bf16x2(s0, s1);
              w.y = pack_bf16x2(s2, s3);
              *reinterpret_cast<uint2*>(p.rs_out + off + j * 32 + 8 * a) = w;
            }
        }
      }
    }
  }
}

// Order of row tiles for a gated consumer: ascending by the stage position at
// which the last 128-row flag of the tile is published (ties by row), so
// compute follows arrival.  Ascending rows when no stage order is given; for
// the reduce epilogue, non-owned rows first and owned rows last.
template <int BM>
__device__ void build_row_perm(const GemmKParams& p, int* row_perm, int* scratch) {
  const int tid = threadIdx.x;
  const int tm = p.tiles_m;
  if (p.perm_mode == kPermArrival) {
    const int nflag = tm * (BM / kFlagRows);
    for (int i = tid; i < nflag; i += kThreads) scratch[p.a_stage_order[i]] = i;  // flag -> position
    __syncthreads();
    for (int i = tid; i < tm; i += kThreads) {
      int key = 0;
      for (int f = 0; f < BM / kFlagRows; ++f) key = max(key, scratch[i * (BM / kFlagRows) + f]);
      scratch[nflag + i] = key;
    }
    __syncthreads();
    for (int i = tid; i < tm; i += kThreads) {
      const int key = scratch[nflag + i];
      int rank = 0;
      for (int j = 0; j < tm; ++j) {
        const int kj = scratch[nflag + j];
        rank += (kj < key) || (kj == key && j < i);
      }
      row_perm[rank] = i;
    }
  } else {  // kPermOwnedLast
    const int own0 = p.rs_own_row0 / BM, nown = p.rs_own_rows / BM;
    for (int i = tid; i < tm; i += kThreads) {
      int r;
      if (i < tm - nown) r = i < own0 ? i : i + nown;
      else r = own0 + (i - (tm - nown));
      row_perm[i] = r;
    }
  }
  __syncthreads();
}

template <int BM, int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmKParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ int row_perm[kMaxTilesM];
  if ((int)blockIdx.x < p.n_prod) {
    producer_role(p, blockIdx.x);
    return;
  }
  int cons = blockIdx.x - p.n_prod;
  // XCD-aware renumbering: workgroups are dealt round-robin to the 8 XCDs,
  // so give each XCD a contiguous run of consumer ids (hence of tiles, which
  // the grouped order keeps close in A rows / B columns) for L2 reuse.
  if (p.xcd_remap) cons = (cons % 8) * (p.n_cons / 8) + cons / 8;
  int* perm = nullptr;
  if (p.perm_mode != kPermNone) {
    build_row_perm<BM>(p, row_perm, reinterpret_cast<int*>(smem));
    perm = row_perm;
  }
  compute_role<BM, EPI>(p, cons, smem, perm);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int BM, int EPI>
static hipError_t launch_t(const GemmKParams& p, hipStream_t stream) {
  const uint32_t lds = TileCfg<BM>::LDS_BYTES;
  static bool attr_set = false;  // per process; the attribute is per function
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, EPI>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((gemm_kernel<BM, EPI>), dim3(p.n_prod + p.n_cons), dim3(kThreads), lds, stream, p);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmKParams& p, int bm, int epi, hipStream_t stream) {
  if (bm == 256) {
    if (epi == kEpiStore) return launch_t<256, kEpiStore>(p, stream);
    if (epi == kEpiReduce) return launch_t<256, kEpiReduce>(p, stream);
    if (epi == kEpiSwiGLU) return launch_t<256, kEpiSwiGLU>(p, stream);
  } else if (bm == 128) {
    if (epi == kEpiStore) return launch_t<128, kEpiStore>(p, stream);
    if (epi == kEpiReduce) return launch_t<128, kEpiReduce>(p, stream);
    if (epi == kEpiSwiGLU) return launch_t<128, kEpiSwiGLU>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mk
