// mk_moe.hip — HBM-bound MoE data movement on gfx950:
//   * permute: expert-contiguous gather of token rows (reference
//     src/dispatch_gemm.cu:106-198 dispatch_fused), 128-bit loads/stores;
//   * combine: deterministic gather of the top-k expert rows of each source
//     token, weighted and summed in fp32 (reference
//     src/dispatch_gemm_glu_combine.cu:736-818 combine_gather_owner; the
//     reference pre-rounds w*y to bf16 in its producer step, here the product
//     stays fp32 because the rows are read in place on the same GPU).
#include "mk_device.h"
#include "mk_internal.h"

namespace mk {

// One workgroup per padded row; padding rows (src_node < 0) are zero-filled.
// With a device row count, rows past it (capacity rows) are left untouched.
__global__ __launch_bounds__(kThreads) void permute_kernel(PermuteKParams p) {
  const int64_t r = blockIdx.x;
  if (p.rows_dev && r >= *p.rows_dev) return;
  const int* pr = p.pull + 3 * r;
  const int src_node = pr[0], src_dev = pr[1], src_tok = pr[2];
  const int64_t vec = p.H / 8;
  uint4* dst = reinterpret_cast<uint4*>(p.post + r * p.H);
  if (src_node < 0 || src_tok < 0) {
    const uint4 z = {0u, 0u, 0u, 0u};
    for (int64_t c = threadIdx.x; c < vec; c += kThreads) dst[c] = z;
    return;
  }
  const int64_t srow = ((int64_t)src_node * p.devs_per_node + src_dev) * p.tokens_per_src + src_tok;
  const uint4* src = reinterpret_cast<const uint4*>(p.tokens + srow * p.H);
  for (int64_t c = threadIdx.x; c < vec; c += kThreads) dst[c] = src[c];
}

hipError_t launch_permute(const PermuteKParams& p, hipStream_t stream) {
  if (p.R_pad == 0) return hipSuccess;
  hipLaunchKernelGGL(permute_kernel, dim3((unsigned)p.R_pad), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

// One workgroup per source token; each thread owns 8 contiguous columns.
// The token's (row, weight) pairs are loaded once per thread, before the
// column loop (at most kMaxSlots of them; more fall back to the slot loop),
// and all of a chunk's row loads are issued before they are summed: the
// kernel is latency-bound, and the dependent owner -> slot -> row -> data
// chain per column chunk made it so.  Sums stay in slot order
// (deterministic, bit-identical to the plain loop).
__global__ __launch_bounds__(kThreads) void combine_kernel(CombineKParams p) {
  constexpr int kMaxSlots = 8;
  const int64_t t = blockIdx.x;
  const int s0 = p.owner_offset[t], s1 = p.owner_offset[t + 1];
  const int n = s1 - s0;
  const int64_t vec = p.H / 8;
  int rows[kMaxSlots];
  float wts[kMaxSlots];
  const bool few = n <= kMaxSlots;
#pragma unroll
  for (int k = 0; k < kMaxSlots; ++k)
    if (few && k < n) rows[k] = p.slot_to_row[s0 + k];
  // a slot whose row is -1 was not produced on this GPU (another owner's
  // combine covers it): it contributes nothing
#pragma unroll
  for (int k = 0; k < kMaxSlots; ++k)
    if (few && k < n) wts[k] = rows[k] >= 0 ? p.row_weight[rows[k]] : 0.f;
  for (int64_t c = threadIdx.x; c < vec; c += kThreads) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto add = [&](float w, const uint4& v) {
      acc[0] += w * bf16_lo(v.x);
      acc[1] += w * bf16_hi(v.x);
      acc[2] += w * bf16_lo(v.y);
      acc[3] += w * bf16_hi(v.y);
      acc[4] += w * bf16_lo(v.z);
      acc[5] += w * bf16_hi(v.z);
      acc[6] += w * bf16_lo(v.w);
      acc[7] += w * bf16_hi(v.w);
    };
    if (few) {
      uint4 v[kMaxSlots];
#pragma unroll
      for (int k = 0; k < kMaxSlots; ++k)
        if (k < n && rows[k] >= 0) v[k] = *reinterpret_cast<const uint4*>(p.y_expert + (int64_t)rows[k] * p.H + c * 8);
#pragma unroll
      for (int k = 0; k < kMaxSlots; ++k)
        if (k < n && rows[k] >= 0) add(wts[k], v[k]);
    } else {
      for (int s = s0; s < s1; ++s) {
        const int row = p.slot_to_row[s];
        if (row < 0) continue;
        add(p.row_weight[row], *reinterpret_cast<const uint4*>(p.y_expert + (int64_t)row * p.H + c * 8));
      }
    }
    // the layer's output is not read again here: nontemporal stores
    // (config 5 layer -7 us against plain stores)
    if (p.out_dtype == 0) {
      float4* o = reinterpret_cast<float4*>(static_cast<float*>(p.y_out) + t * p.H + c * 8);
      __builtin_nontemporal_store(f32x4{acc[0], acc[1], acc[2], acc[3]}, reinterpret_cast<f32x4*>(o));
      __builtin_nontemporal_store(f32x4{acc[4], acc[5], acc[6], acc[7]}, reinterpret_cast<f32x4*>(o) + 1);
    } else {
      uint4 w;
      w.x = pack_bf16x2(acc[0], acc[1]);
      w.y = pack_bf16x2(acc[2], acc[3]);
      w.z = pack_bf16x2(acc[4], acc[5]);
      w.w = pack_bf16x2(acc[6], acc[7]);
      typedef uint32_t u4 __attribute__((ext_vector_type(4)));
      __builtin_nontemporal_store(u4{w.x, w.y, w.z, w.w}, reinterpret_cast<u4*>(static_cast<uint16_t*>(p.y_out) + t * p.H + c * 8));
    }
  }
}

hipError_t launch_combine(const CombineKParams& p, hipStream_t stream) {
  if (p.num_tokens == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)p.num_tokens), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

// One workgroup per 128-row block: count rows with a real source token.
__global__ __launch_bounds__(128) void tile_rows_kernel(const int* pull, int64_t R_pad, int* rb_rows) {
  const int64_t r = (int64_t)blockIdx.x * 128 + threadIdx.x;
  const int real = (r < R_pad && pull[3 * r] >= 0) ? 1 : 0;
  const int n = __syncthreads_count(real);
  if (threadIdx.x == 0) rb_rows[blockIdx.x] = n;
}

hipError_t launch_tile_rows(const int* pull, int64_t R_pad, int* rb_rows, hipStream_t stream) {
  if (R_pad == 0) return hipSuccess;
  hipLaunchKernelGGL(tile_rows_kernel, dim3((unsigned)((R_pad + 127) / 128)), dim3(128), 0, stream, pull, R_pad, rb_rows);
  return hipGetLastError();
}

__global__ void fill_i32_kernel(int* dst, int64_t n, int value) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = value;
}

// Rows of `owner` only; a slot outside [0, cap) is skipped and reported.
__global__ void invert_slots_kernel(const int* row_to_slot, const int* row_to_owner, int64_t R_pad, int owner,
                                    int64_t cap, int* slot_to_row, uint32_t* err) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R_pad || row_to_owner[r] != owner) return;
  const int s = row_to_slot[r];
  if (s >= 0 && s < cap) slot_to_row[s] = (int)r;
  else if (err) __hip_atomic_fetch_or(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

hipError_t launch_invert_slots(const int* row_to_slot, const int* row_to_owner, int64_t R_pad, int owner,
                               int64_t cap, int* slot_to_row, uint32_t* err, hipStream_t stream) {
  // a fill kernel, not hipMemsetAsync, so the pair can be recorded in a graph
  if (cap > 0)
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((cap + 255) / 256)), dim3(256), 0, stream, slot_to_row, cap, -1);
  if (R_pad > 0)
    hipLaunchKernelGGL(invert_slots_kernel, dim3((unsigned)((R_pad + 255) / 256)), dim3(256), 0, stream, row_to_slot,
                       row_to_owner, R_pad, owner, cap, slot_to_row, err);
  return hipGetLastError();
}

}  // namespace mk
