// mk_device.h — device-side vocabulary shared by the libmk kernels (gfx950).
//
// * bf16 storage is uint16_t; MFMA operands are 8 x __bf16 vectors.
// * Flags are epoch-stamped 32-bit words.  Data is written through to agent
//   scope (write-through stores, then s_waitcnt vmcnt(0)) and the flag is a
//   relaxed agent-scope store; consumers poll with relaxed agent-scope loads
//   and acquire-fence once the epoch is seen.  This is the ordering contract
//   of the reference's comm::atomic_u32 release_store_gpu / acquire_load_gpu
//   pair (reference include/comm/atomic_u32.cuh:33-95) expressed with the
//   HIP memory model (publish_flag is the plain release store, for data
//   written without write-through).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 wavefronts of 64 (permute / combine kernels)
constexpr int kFlagRows = 128; // flag granularity

// Buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Wait until every flag addr(0) .. addr(n-1) has reached `epoch`
// (wrap-safe).  Each round loads all flags still pending at once (relaxed
// agent-scope loads issued back to back: one memory latency per round, not
// per flag), in chunks of kChunk (<= 32); rounds are spaced by s_sleep with a growing
// interval (64 .. 1024 cycles), so a few hundred waiting workgroups do not
// flood the L2 the producers are writing through.  One acquire fence
// follows.  Returns false (and sets bit 0 of *err) after `limit` rounds of
// one chunk when limit != 0.
template <int kChunk, class Addr>
__device__ __forceinline__ bool wait_flags(Addr addr, int n, uint32_t epoch, uint32_t limit, uint32_t* err) {
  static_assert(kChunk >= 1 && kChunk <= 32, "flag chunk");
  for (int base = 0; base < n; base += kChunk) {
    const int m = min(n - base, kChunk);
    uint32_t pending = m == 32 ? ~0u : (1u << m) - 1u;
    uint32_t polls = 0;
    while (true) {
      uint32_t v[kChunk];
#pragma unroll
      for (int f = 0; f < kChunk; ++f)
        if ((pending >> f) & 1u) v[f] = __hip_atomic_load(addr(base + f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int f = 0; f < kChunk; ++f)
        if (((pending >> f) & 1u) && (int32_t)(v[f] - epoch) >= 0) pending &= ~(1u << f);
      if (!pending) break;
      if (limit != 0 && ++polls >= limit) {
        if (err) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
      if (polls < 8) __builtin_amdgcn_s_sleep(1);
      else if (polls < 64) __builtin_amdgcn_s_sleep(4);
      else __builtin_amdgcn_s_sleep(16);
      if (limit == 0) ++polls;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return true;
}

__device__ __forceinline__ void publish_flag(uint32_t* flag, uint32_t epoch) {
  __hip_atomic_store(flag, epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// s_waitcnt vmcnt(0), other counters untouched (gfx9 encoding).
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Write-through staging copy of `nvec` 16-byte units, `NT` threads, U loads
// in flight per thread.  Loads are nontemporal (the source is read once);
// stores are buffer stores with SC1: each store is coherent at agent scope
// (the form the AMDGPU memory model gives a relaxed agent-scope atomic
// store: written through the XCD's L2).  They carry no nontemporal hint:
// the compute workgroups read the staged rows soon after, and letting the
// caches keep them measured 14 us faster per config-2 launch than SC1|NT.
// Publication protocol built on it: every wave waits vmcnt(0) for its own
// stores (after which they are performed at agent scope), a workgroup
// barrier, then one thread's relaxed agent-scope atomics publish.  This is
// the release sequence of the memory model minus its L2 write-back
// (buffer_wbl2), which is only needed for data written without SC1 — and
// that write-back flushes every dirty line of the XCD's L2, which cost the
// staging ~15 % of the launch when it ran once per published batch.
template <int NT, int U>
__device__ __forceinline__ void copy_wt(const void* src, void* dst, int64_t nvec) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4* s = static_cast<const u32x4*>(src);
  const __amdgpu_buffer_rsrc_t r = make_rsrc(dst, (uint32_t)(nvec * 16));
  constexpr int kCpolSc1 = 0x10;  // gfx940+ cache policy: SC1
  int64_t base = threadIdx.x;
  for (; base + (int64_t)(U - 1) * NT < nvec; base += (int64_t)U * NT) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(s + base + u * NT);
#pragma unroll
    for (int u = 0; u < U; ++u)
      __builtin_amdgcn_raw_buffer_store_b128(v[u], r, (int)((base + u * NT) * 16), 0, kCpolSc1);
  }
  for (; base < nvec; base += NT)
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_nontemporal_load(s + base), r, (int)(base * 16), 0, kCpolSc1);
}

}  // namespace mk
