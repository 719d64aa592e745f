// mk_moe_index.hip — MoE routing index tables built on the GPU.
//
// Same tables, bit for bit, as the host builder mk_moe_build_indices (which
// restates the reference's host-side Python builders
// bench/dispatch_gemm_bench.py:127-188 and
// bench/dispatch_gemm_glu_combine_bench.py:222-293, 511-527), from top-k ids
// and gates already in device memory, with no host round trip:
//   * rows grouped by local expert (ascending), each expert padded to a
//     multiple of row_block; inside an expert, entries (t, k) in ascending
//     t*topk + k order — a stable counting sort of the routed entries by
//     expert;
//   * pull_indices (0, 0, t) for a routed row, (-1, -1, -1) for padding;
//   * the gather CSR: owner_offset = prefix over tokens of their routed
//     entries, slots handed out in row order (so a token's slots follow its
//     rows' expert order), and its inverse slot_to_row.
//
// Kernels (one stream, in order):
//   count   per 256-entry chunk, per-expert counts            -> hist[e][chunk]
//           per 256 tokens, routed entries                     -> tok[t]
//   plan    one block: per-expert totals and chunk prefixes, padded expert
//           offsets, R and R_pad, per-expert tables           -> base[e][chunk]
//           exclusive prefix of tok                            -> owner_offset
//   scatter per chunk: stable rank within the chunk, row, slot -> routed rows
//           per 256 rows < R_pad: expert of the row, padding rows, row-block tables
#include <algorithm>

#include "../../include/mk.h"
#include "mk_internal.h"

namespace mk {

constexpr int kChunk = 256;  // routed entries per count / scatter block

struct IndexKParams {
  const int32_t* ids;
  const float* gates;
  int T, topk, e0, n_local, row_block;
  int64_t cap;       // rows the row tables hold
  int nchunks;
  int* hist;         // [n_local][nchunks] counts, then row bases
  int* exp_off;      // [n_local + 1] padded row offset of each expert
  int* exp_cnt;      // [n_local] routed rows of each expert
  int* tok;          // [T] routed entries per token
  int64_t* sizes;    // [2] R, R_pad
  mk_moe_index out;
};

__device__ __forceinline__ int local_expert(const IndexKParams& p, int64_t i) {
  const int e = p.ids[i] - p.e0;
  return (e >= 0 && e < p.n_local) ? e : -1;
}

// Block b: the per-expert histogram of entry chunk b (b < nchunks) and the
// routed-entry count of tokens 256b .. 256b+255 (the tokens pass, merged
// into the same launch).
__global__ __launch_bounds__(kChunk) void count_kernel(IndexKParams p) {
  extern __shared__ int h[];
  if ((int)blockIdx.x < p.nchunks) {
    for (int e = threadIdx.x; e < p.n_local; e += kChunk) h[e] = 0;
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * kChunk + threadIdx.x;
    if (i < (int64_t)p.T * p.topk) {
      const int e = local_expert(p, i);
      if (e >= 0) atomicAdd(&h[e], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < p.n_local; e += kChunk) p.hist[(int64_t)e * p.nchunks + blockIdx.x] = h[e];
  }
  const int t = blockIdx.x * kChunk + threadIdx.x;
  if (t < p.T) {
    int c = 0;
    for (int k = 0; k < p.topk; ++k) c += local_expert(p, (int64_t)t * p.topk + k) >= 0;
    p.tok[t] = c;
  }
}

// Block-wide exclusive scan of one value per thread (NT threads), total out:
// inclusive prefix sums inside each wave by shuffles, the wave totals
// scanned by the first wave, two workgroup barriers in all.  `s` holds at
// least NT / 64 + 1 ints.
template <int NT>
__device__ int block_exclusive_scan(int v, int* s, int& total) {
  constexpr int W = NT / 64;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) s[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    const int wt = lane < W ? s[lane] : 0;
    int wi = wt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(wi, d, 64);
      if (lane >= d) wi += y;
    }
    if (lane < W) s[lane] = wi - wt;       // exclusive prefix of the wave totals
    if (lane == W - 1) s[W] = wi;          // block total
  }
  __syncthreads();
  total = s[W];
  const int r = s[wave] + incl - v;
  __syncthreads();  // s is reused by the next scan
  return r;
}

constexpr int kPlanThreads = 1024;
constexpr int kPlanSteps = 4;  // chunk counts of one expert loaded together: 64 x kPlanSteps per wave
constexpr int kTokSeg = 8;     // token counts per thread in one block scan (kPlanThreads x kTokSeg tokens)

// One workgroup; a chain of dependent steps, so every step issues its loads
// together: the first token segment is loaded at kernel start (the token
// scan does not depend on the expert work), each wave loads up to
// 64 x kPlanSteps chunk counts of an expert before scanning them, and the
// per-expert totals go through LDS as well as global memory.
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(IndexKParams p) {
  __shared__ int s[kPlanThreads];
  __shared__ int cnt_s[kPlanThreads];  // exp_cnt of experts below kPlanThreads
  __shared__ int carry;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // token pass 0: tokens t0 .. t0 + n, thread i holding `per` consecutive ones
  const int n0 = min(p.T, kPlanThreads * kTokSeg);
  const int per0 = (n0 + kPlanThreads - 1) / kPlanThreads;
  int tv[kTokSeg];
#pragma unroll
  for (int k = 0; k < kTokSeg; ++k) {
    const int t = threadIdx.x * per0 + k;
    tv[k] = (k < per0 && t < n0) ? p.tok[t] : 0;
  }
  // per expert: totals, and the exclusive prefix over chunks (in place);
  // one wave per expert, wave prefix sums by shuffles
  for (int e = wave; e < p.n_local; e += kPlanThreads / 64) {
    int* h = p.hist + (int64_t)e * p.nchunks;
    int carry_e = 0;
    for (int c0 = 0; c0 < p.nchunks; c0 += 64 * kPlanSteps) {
      int v[kPlanSteps];
#pragma unroll
      for (int k = 0; k < kPlanSteps; ++k) {
        const int c = c0 + 64 * k + lane;
        v[k] = c < p.nchunks ? h[c] : 0;
      }
#pragma unroll
      for (int k = 0; k < kPlanSteps; ++k) {
        const int c = c0 + 64 * k + lane;
        int incl = v[k];
        for (int d = 1; d < 64; d <<= 1) {
          const int y = __shfl_up(incl, d, 64);
          if (lane >= d) incl += y;
        }
        if (c < p.nchunks) h[c] = carry_e + incl - v[k];
        carry_e += __shfl(incl, 63, 64);
      }
    }
    if (lane == 0) {
      p.exp_cnt[e] = carry_e;
      if (e < kPlanThreads) cnt_s[e] = carry_e;
    }
  }
  __syncthreads();
  // padded expert offsets: exclusive scan over experts, kPlanThreads at a time
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  int64_t routed = 0;
  for (int e0 = 0; e0 < p.n_local; e0 += kPlanThreads) {
    const int e = e0 + threadIdx.x;
    const int cnt = e < p.n_local ? (e < kPlanThreads ? cnt_s[e] : p.exp_cnt[e]) : 0;
    const int padded = (cnt + p.row_block - 1) / p.row_block * p.row_block;
    int tot;
    const int ex = block_exclusive_scan<kPlanThreads>(padded, s, tot);
    if (e < p.n_local) {
      p.exp_off[e] = carry + ex;
      if (e < kPlanThreads) cnt_s[e] = carry + ex;  // now the expert's row offset
      if (p.out.padded_tokens_per_expert) p.out.padded_tokens_per_expert[e] = padded;
      if (p.out.local_rb_per_expert) p.out.local_rb_per_expert[e] = cnt / p.row_block;
    }
    int rtot;
    block_exclusive_scan<kPlanThreads>(cnt, s, rtot);
    routed += rtot;
    __syncthreads();
    if (threadIdx.x == 0) carry += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.exp_off[p.n_local] = carry;
    p.sizes[0] = routed;
    p.sizes[1] = carry;
  }
  __syncthreads();
  // chunk prefixes become absolute row bases
  for (int e = wave; e < p.n_local; e += kPlanThreads / 64) {
    int* h = p.hist + (int64_t)e * p.nchunks;
    const int off = e < kPlanThreads ? cnt_s[e] : p.exp_off[e];
    for (int c = lane; c < p.nchunks; c += 64) h[c] += off;
  }
  // token CSR offsets: exclusive prefix of the per-token counts (the
  // offsets pass, merged into the same launch), kPlanThreads x kTokSeg
  // tokens per block scan
  int tcarry = 0;
  for (int t0 = 0; t0 < p.T; t0 += kPlanThreads * kTokSeg) {
    const int n = min(p.T - t0, kPlanThreads * kTokSeg);
    const int per = (n + kPlanThreads - 1) / kPlanThreads;
    const int tb = t0 + threadIdx.x * per;
    int v[kTokSeg], sum = 0;
#pragma unroll
    for (int k = 0; k < kTokSeg; ++k) {
      v[k] = t0 == 0 ? tv[k] : ((k < per && tb + k < t0 + n) ? p.tok[tb + k] : 0);
      sum += v[k];
    }
    int tot;
    const int ex = block_exclusive_scan<kPlanThreads>(sum, s, tot);
    if (p.out.owner_offset) {
      int run = tcarry + ex;
#pragma unroll
      for (int k = 0; k < kTokSeg; ++k)
        if (k < per && tb + k < t0 + n) {
          p.out.owner_offset[tb + k] = run;
          run += v[k];
        }
    }
    tcarry += tot;
  }
  if (threadIdx.x == 0 && p.out.owner_offset) p.out.owner_offset[p.T] = tcarry;
}

// Block b: the routed rows of entry chunk b (b < nchunks), then rows
// 256b .. 256b+255 of the padded table (the padding pass, merged into the
// same launch; it writes every row's expert and the padding rows only, so
// the two parts never write the same field).
__global__ __launch_bounds__(kChunk) void scatter_kernel(IndexKParams p) {
  extern __shared__ int wcnt[];  // [kChunk / 64 waves][n_local]: per-wave counts of each expert
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const mk_moe_index& o = p.out;
  if ((int)blockIdx.x < p.nchunks) {
    const int64_t i = (int64_t)blockIdx.x * kChunk + threadIdx.x;
    const int e = i < (int64_t)p.T * p.topk ? local_expert(p, i) : -1;
    for (int x = lane; x < p.n_local; x += 64) wcnt[wave * p.n_local + x] = 0;
    // stable rank among the chunk's earlier entries of the same expert:
    // inside the wave by one ballot per distinct expert, plus the counts
    // of the earlier waves
    int rank = 0;
    uint64_t pending = __ballot(e >= 0);
    while (pending) {
      const int el = __shfl(e, __builtin_ctzll(pending), 64);
      const uint64_t m = __ballot(e == el);
      if (e == el) rank = __popcll(m & ((1ull << lane) - 1ull));
      if (lane == 0) wcnt[wave * p.n_local + el] = __popcll(m);
      pending &= ~m;
    }
    __syncthreads();
    if (e >= 0) {
      for (int w = 0; w < wave; ++w) rank += wcnt[w * p.n_local + e];
      const int64_t row = (int64_t)p.hist[(int64_t)e * p.nchunks + blockIdx.x] + rank;
      const int t = (int)(i / p.topk), k = (int)(i % p.topk);
      // slot: the token's routed entries in row order = (expert, k) order
      int before = 0;
      for (int k2 = 0; k2 < p.topk; ++k2) {
        const int e2 = local_expert(p, (int64_t)t * p.topk + k2);
        before += e2 >= 0 && (e2 < e || (e2 == e && k2 < k));
      }
      if (row < p.cap) {  // past the capacity: sizes reports R_pad > cap
        if (o.pull_indices) {
          o.pull_indices[3 * row + 0] = 0;
          o.pull_indices[3 * row + 1] = 0;
          o.pull_indices[3 * row + 2] = t;
        }
        if (o.row_weight) o.row_weight[row] = p.gates[i];
        if (o.row_to_owner) o.row_to_owner[row] = 0;
        if (o.owner_offset) {
          const int slot = o.owner_offset[t] + before;
          if (o.row_to_slot) o.row_to_slot[row] = slot;
          if (o.slot_to_row) o.slot_to_row[slot] = (int32_t)row;
        }
      }
    }
  }
  const int64_t r = (int64_t)blockIdx.x * kChunk + threadIdx.x;
  const int64_t R_pad = p.sizes[1];
  if (r >= R_pad || r >= p.cap) return;
  // expert of row r: last e with exp_off[e] <= r (binary search)
  int lo = 0, hi = p.n_local - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (p.exp_off[mid] <= r) lo = mid;
    else hi = mid - 1;
  }
  const int e = lo;
  const int64_t ie = r - p.exp_off[e];
  const int cnt = p.exp_cnt[e];
  if (o.row_expert) o.row_expert[r] = e;
  if (ie >= cnt) {
    if (o.pull_indices) {
      o.pull_indices[3 * r + 0] = -1;
      o.pull_indices[3 * r + 1] = -1;
      o.pull_indices[3 * r + 2] = -1;
    }
    if (o.row_weight) o.row_weight[r] = 0.f;
    if (o.row_to_slot) o.row_to_slot[r] = 0;
    if (o.row_to_owner) o.row_to_owner[r] = -1;
  }
  if (r % p.row_block == 0) {
    const int64_t b = r / p.row_block;
    if (o.rb_expert) o.rb_expert[b] = e;
    if (o.rb_rows) o.rb_rows[b] = (int)max((int64_t)0, min((int64_t)p.row_block, (int64_t)cnt - ie));
  }
}

int64_t index_workspace_bytes(int T, int topk, int n_local) {
  const int64_t nchunks = ((int64_t)T * topk + kChunk - 1) / kChunk;
  const int64_t ints = (int64_t)n_local * (nchunks > 0 ? nchunks : 1) + 2 * (int64_t)n_local + 1 + T;
  return (ints * 4 + 255) / 256 * 256;
}

hipError_t launch_build_indices(const int32_t* ids, const float* gates, int T, int topk, int e0, int n_local,
                                int row_block, int64_t cap, void* ws, int64_t* sizes, const mk_moe_index& out,
                                hipStream_t stream) {
  IndexKParams p;
  p.ids = ids;
  p.gates = gates;
  p.T = T; p.topk = topk; p.e0 = e0; p.n_local = n_local; p.row_block = row_block;
  p.cap = cap;
  p.nchunks = (int)(((int64_t)T * topk + kChunk - 1) / kChunk);
  const int nch = p.nchunks > 0 ? p.nchunks : 1;
  int* w = static_cast<int*>(ws);
  p.hist = w;
  p.exp_off = w + (int64_t)n_local * nch;
  p.exp_cnt = p.exp_off + n_local + 1;
  p.tok = p.exp_cnt + n_local;
  p.sizes = sizes;
  p.out = out;
  // (no routed entries: plan sees nchunks = 0 and empty experts)
  const int64_t tblocks = ((int64_t)T + kChunk - 1) / kChunk;
  const int64_t g1 = std::max<int64_t>(p.nchunks, tblocks);
  if (g1 > 0)
    hipLaunchKernelGGL(count_kernel, dim3((unsigned)g1), dim3(kChunk), n_local * sizeof(int), stream, p);
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p);
  const int64_t g3 = std::max<int64_t>(p.nchunks, (cap + kChunk - 1) / kChunk);
  if (g3 > 0)
    hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)g3), dim3(kChunk), (kChunk / 64) * n_local * sizeof(int), stream,
                       p);
  return hipGetLastError();
}

}  // namespace mk
