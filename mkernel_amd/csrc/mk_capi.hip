// mk_capi.hip — the extern "C" boundary of libmk (declared in include/mk.h):
// argument and shape validation, persistent-grid sizing and role split, and
// the host-side MoE routing index build.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mk.h"
#include "mk_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  g_err = std::string(where) + ": " + hipGetErrorString(e);
  return (int)e;
}

struct DevInfo {
  int cus = 0;
  bool ok = false;
};

// Per-device properties, read once per device.
int device_info(DevInfo* out) {
  static std::mutex mu;
  static std::vector<DevInfo> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1);
  if (!cache[dev].ok) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      return fail(MK_EDEVICE, "libmk is built for gfx950 only; device %d is %s", dev, prop.gcnArchName);
    cache[dev].cus = prop.multiProcessorCount;
    cache[dev].ok = true;
  }
  *out = cache[dev];
  return MK_OK;
}

// Persistent grid size: 0 = every CU.  More workgroups than CUs is refused:
// the flag waits, cooperative staging and the K-split exchange all assume
// that every workgroup of the launch is resident at once (one per CU).
int grid_total(int num_cus, const DevInfo& d, const char* fn, int* total) {
  if (num_cus < 0 || num_cus > d.cus)
    return fail(MK_EINVAL, "%s: num_cus=%d must be 0 (every CU) or at most the device's %d CUs", fn, num_cus, d.cus);
  *total = num_cus > 0 ? num_cus : d.cus;
  return MK_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

void fill_common(mk::GemmKParams& p) {
  std::memset(&p, 0, sizeof p);
  p.group_m = 8;
  p.waves = 8;
}

// Split `total` workgroups into producers + consumers; enable the XCD remap
// when both counts are multiples of the 8 XCDs.
void set_grid(mk::GemmKParams& p, int total, int n_prod, int ntiles) {
  p.n_prod = n_prod;
  p.n_cons = std::max(1, std::min(total - n_prod, ntiles));
  p.xcd_remap = (p.n_cons % 8 == 0 && p.n_prod % 8 == 0) ? 1 : 0;
}

int check_gemm_shape(int64_t M, int64_t N, int64_t K, int bm, int64_t lda = 0, int64_t ldb = 0) {
  if (M <= 0 || N <= 0 || K <= 0) return fail(MK_ESHAPE, "M, N, K must be positive (got %lld, %lld, %lld)",
                                              (long long)M, (long long)N, (long long)K);
  if (M % bm) return fail(MK_ESHAPE, "M=%lld must be a multiple of %d", (long long)M, bm);
  if (N % 256) return fail(MK_ESHAPE, "N=%lld must be a multiple of 256", (long long)N);
  if (K % 32) return fail(MK_ESHAPE, "K=%lld must be a multiple of 32", (long long)K);
  if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30)) return fail(MK_ESHAPE, "dimension too large");
  // The K loop addresses operands through buffer descriptors with 32-bit
  // offsets: one row tile of A (whose padding rows use offsets from 2^31
  // up, past the window) and all of B (one expert's B for grouped GEMMs).
  if (lda <= 0) lda = K;
  if (ldb <= 0) ldb = N;
  if ((int64_t)bm * lda * 2 >= (1LL << 31))
    return fail(MK_ESHAPE, "a %d-row tile of A (lda=%lld) must span less than 2 GiB", bm, (long long)lda);
  if (K * ldb * 2 >= (1LL << 32))
    return fail(MK_ESHAPE, "B (K=%lld x ldb=%lld) must be smaller than 4 GiB", (long long)K, (long long)ldb);
  return MK_OK;
}

constexpr int64_t kSplitTileBytes = 256 * 256 * 4;  // one fp32 partial tile (BM x BN <= 256 x 256)
constexpr int64_t kSplitFlagBytes = 4096;           // flag words at the start of the workspace
// The last 64 bytes of the flag area hold the claim word of co-resident
// staging (epoch-stamped, never reset); K-split flags use the bytes before.
constexpr int64_t kClaimOffset = kSplitFlagBytes - 64;

int64_t split_ws_bytes(int cus) { return kSplitFlagBytes + (int64_t)cus * kSplitTileBytes; }

// K-split plan for the tail round: with R = tiles % n_cons tiles left for a
// partial last round, split each of them s = min(4, n_cons / R) ways along
// K so that R*s workgroups share the round.  The workspace holds the flag
// words at a fixed offset (so every plan finds them zeroed) followed by
// R*(s-1) < n_cons <= CUs partial tiles, which split_ws_bytes covers.
void plan_split(mk::GemmKParams& p, int bm, void* ws, int64_t ws_bytes, int bn = 256) {
  const int ntiles = p.tiles_m * p.tiles_n;
  const int R = ntiles % p.n_cons;
  if (!ws || R == 0 || p.waves != 8) return;
  if (p.perm_mode != mk::kPermNone && ntiles > mk::kMaxSplitListTiles) return;
  int s = std::min(4, p.n_cons / R);
  s = std::min(s, (p.K / 32) / 4);  // keep every part at >= 4 K stages
  if (s < 2) return;
  const int64_t parts = (int64_t)R * (s - 1);
  if (parts * 4 > kClaimOffset || kSplitFlagBytes + parts * bm * bn * 4 > ws_bytes) return;
  p.sk_flags = static_cast<uint32_t*>(ws);
  p.sk_ws = reinterpret_cast<float*>(static_cast<char*>(ws) + kSplitFlagBytes);
  p.sk_full = ntiles - R;
  p.sk_split = s;
}

int check_ws(const void* ws, int64_t bytes, const char* fn) {
  if (ws && (bytes < 0 || (reinterpret_cast<uintptr_t>(ws) & 255u)))
    return fail(MK_EINVAL, "%s: split_ws must be 256-byte aligned with a non-negative size", fn);
  return MK_OK;
}

// num_producers <= -3 asks for the co-resident staging kernel with
// -2 - num_producers one-wave workgroups per CU (1..4).  Under graph capture
// the fork/join would become two graph branches whose order the replay does
// not fix, so the launch stages cooperatively instead (*waves = 0).
int costage_request(int gated, int num_producers, const void* split_ws, int64_t split_ws_bytes, void* stream,
                    const char* fn, int* waves) {
  *waves = (gated && num_producers <= -3) ? -2 - num_producers : 0;
  if (!*waves) return MK_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t ce = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cap);
  if (ce != hipSuccess) return hip_fail(ce, "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone) {
    *waves = 0;
    return MK_OK;
  }
  if (!split_ws || split_ws_bytes < kSplitFlagBytes)
    return fail(MK_EINVAL, "%s: co-resident staging keeps its claim word in split_ws, which is NULL or short", fn);
  return MK_OK;
}

}  // namespace

namespace mk {
hipError_t launch_build_indices(const int32_t* ids, const float* gates, int T, int topk, int e0, int n_local,
                                int row_block, int64_t cap, void* ws, int64_t* sizes, const mk_moe_index& out,
                                hipStream_t stream);
}

// ---------------------------------------------------------------------------
// mk_ag_gemm_noalloc: mk_ag_gemm with its scratch (the K-split workspace and
// the cooperative-staging piece counters) in `scratch`, a static device
// array: one copy per GPU, held until the process ends, so the call makes no
// allocation.  Layout: [K-split flag words, 4 KB][kNoAllocTiles fp32
// 256x256 partial tiles][kNoAllocCounters piece counters].  Host code never
// uses the symbol's name as an address: the device address comes from
// hipGetSymbolAddress, once per device, and only that pointer is passed on.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kNoAllocTiles = 128;        // K-split partial tiles (32 MB)
constexpr int64_t kNoAllocCounters = 16384;   // one per 128-row block: M <= 2^21 rows
constexpr int64_t kNoAllocSplitBytes = kSplitFlagBytes + kNoAllocTiles * kSplitTileBytes;
constexpr int64_t kNoAllocBytes = kNoAllocSplitBytes + kNoAllocCounters * 4;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // device address of `scratch`, per device

// Device address of this device's `scratch` (looked up on the first call on
// each device, with that device current).
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(MK_EDEVICE, "hipGetSymbolAddress(scratch) returned no address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MK_OK;
}

// Zeroes the K-split flag words and the first n_counters piece counters (a
// kernel rather than hipMemsetAsync, so the call can be graph-captured).
__global__ void clear_scratch_kernel(uint32_t* split_flags, int n_flags, uint32_t* counters, int n_counters) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_flags) split_flags[i] = 0u;
  if (i < n_counters) counters[i] = 0u;
}
}  // namespace

extern "C" {

const char* mk_last_error_string(void) { return g_err.c_str(); }

int32_t mk_abi_version(void) { return 7; }

int mk_epoch_advance(uint32_t* epoch_ptr, void* stream) {
  if (!epoch_ptr) return fail(MK_EINVAL, "mk_epoch_advance: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  hipError_t e = mk::launch_epoch_advance(epoch_ptr, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_epoch_advance launch");
}

int mk_probe_mfma_ceiling(int64_t iters, int32_t num_wg, float* sink, uint64_t* clocks, void* stream) {
  if (!sink || !clocks) return fail(MK_EINVAL, "mk_probe_mfma_ceiling: null argument");
  if (iters <= 0 || num_wg <= 0) return fail(MK_EINVAL, "mk_probe_mfma_ceiling: iters and num_wg must be positive");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  hipError_t e = mk::launch_mfma_ceiling(iters, num_wg, 12345u, sink, clocks, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_probe_mfma_ceiling launch");
}

int32_t mk_probe_threads(void) { return mk::probe_threads(); }

int32_t mk_device_cu_count(void) {
  DevInfo d;
  if (device_info(&d) != MK_OK) return 0;
  return d.cus;
}

int64_t mk_query_workspace_bytes(int32_t which, int64_t M, int64_t N, int64_t K) {
  (void)which; (void)M; (void)N; (void)K;
  DevInfo d;
  if (device_info(&d) != MK_OK) return -1;
  return split_ws_bytes(d.cus);
}

int mk_gemm(const mk_gemm_args* a, void* stream) {
  if (!a || !a->A || !a->B || !a->C) return fail(MK_EINVAL, "mk_gemm: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  int bm = a->tile_m;
  if (bm == 0) {
    // 256-row tiles unless 128-row ones fit in one round: a partial round
    // of 256-row tiles (spread over the XCDs) beats two rounds of 128-row
    // ones (4352x2048x8192: 137 vs 176 us; 4096x3584x8192: 188 vs 264 us),
    // while one round of 128-row tiles beats a half-empty 256-row round
    // (4096x2048x8192: 137 vs 145 us; 2048^2 x 8192: 116 vs 128 us).
    const int64_t t256 = (a->M % 256 == 0) ? (a->M / 256) * (a->N / 256) : 0;
    bm = (2 * t256 > d.cus) ? 256 : 128;
  }
  if (bm != 128 && bm != 256) return fail(MK_EINVAL, "mk_gemm: tile_m must be 0, 128 or 256");
  if (a->waves != 0 && a->waves != 4 && a->waves != 8) return fail(MK_EINVAL, "mk_gemm: waves must be 0, 4 or 8");
  if (int rc = check_gemm_shape(a->M, a->N, a->K, bm, a->lda, a->ldb)) return rc;
  if (a->lda < a->K || a->ldb < a->N || a->ldc < a->N || (a->lda | a->ldb | a->ldc) % 8)
    return fail(MK_ESHAPE, "mk_gemm: leading dimensions must cover the row and be multiples of 8");
  if (!aligned16(a->A) || !aligned16(a->B) || !aligned16(a->C))
    return fail(MK_EINVAL, "mk_gemm: pointers must be 16-byte aligned");
  mk::GemmKParams p;
  fill_common(p);
  p.A = static_cast<const uint16_t*>(a->A);
  p.B = static_cast<const uint16_t*>(a->B);
  p.C = static_cast<uint16_t*>(a->C);
  p.lda = a->lda; p.ldb = a->ldb; p.ldc = a->ldc;
  p.M = (int)a->M; p.N = (int)a->N; p.K = (int)a->K;
  p.tiles_m = (int)(a->M / bm);
  p.tiles_n = (int)(a->N / 256);
  int total;
  if (int rc = grid_total(a->num_cus, d, "mk_gemm", &total)) return rc;
  set_grid(p, total, 0, p.tiles_m * p.tiles_n);
  if (a->waves) p.waves = a->waves;
  if (int rc = check_ws(a->split_ws, a->split_ws_bytes, "mk_gemm")) return rc;
  plan_split(p, bm, a->split_ws, a->split_ws_bytes);
  hipError_t e = mk::launch_gemm(p, bm, mk::kEpiStore, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_gemm launch");
}

}  // extern "C"

namespace {
// Validates mk_ag_gemm's arguments and fills the launch: every refusal
// happens here, before anything is queued.  *costage_waves > 0 selects the
// co-resident staging kernel (that many one-wave workgroups).
int prepare_ag(const mk_ag_gemm_args* a, void* stream, mk::GemmKParams& p, int* costage_out) {
  if (!a || !a->A_full || !a->B || !a->C) return fail(MK_EINVAL, "mk_ag_gemm: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  const int bm = 256;
  if (int rc = check_gemm_shape(a->M, a->N, a->K, bm)) return rc;
  const int64_t nflags = a->M / 128;
  if (a->gated) {
    if (!a->flags) return fail(MK_EINVAL, "mk_ag_gemm: gated launch needs flags");
    if (a->epoch == 0 && !a->epoch_ptr) return fail(MK_EINVAL, "mk_ag_gemm: epoch 0 is reserved (flags start at 0)");
    if (a->stage_order && a->M / bm > mk::kMaxTilesM)
      return fail(MK_ESHAPE, "mk_ag_gemm: arrival-ordered schedule supports at most %d row tiles", mk::kMaxTilesM);
    if (nflags + a->M / bm > 8192)
      return fail(MK_ESHAPE, "mk_ag_gemm: too many flags for the schedule scratch");
  }
  if (a->num_producers < -6) return fail(MK_EINVAL, "mk_ag_gemm: num_producers must be >= -6");
  if (a->gated && a->num_producers != 0 && !a->A_shards)
    return fail(MK_EINVAL, "mk_ag_gemm: staging needs A_shards");
  const bool coop = a->gated && a->num_producers < 0;
  // num_producers <= -3: co-resident staging kernel, -2 - num_producers
  // one-wave workgroups per CU beside the GEMM
  int costage_waves = 0;
  if (int rc = costage_request(a->gated, a->num_producers, a->split_ws, a->split_ws_bytes, stream, "mk_ag_gemm",
                               &costage_waves))
    return rc;
  if (coop && !a->stage_counters) return fail(MK_EINVAL, "mk_ag_gemm: cooperative staging needs stage_counters");
  int total;
  if (int rc = grid_total(a->num_cus, d, "mk_ag_gemm", &total)) return rc;
  const int n_prod = (a->gated && a->num_producers > 0) ? a->num_producers : 0;
  if (n_prod >= total) return fail(MK_EINVAL, "mk_ag_gemm: num_producers (%d) leaves no compute workgroups", n_prod);
  if (a->n_present < 0 || a->n_present > nflags)
    return fail(MK_EINVAL, "mk_ag_gemm: n_present=%d must be in [0, M/128]", a->n_present);
  if (a->n_present > 0 && !a->stage_order)
    return fail(MK_EINVAL, "mk_ag_gemm: n_present needs stage_order (the present blocks are its first entries)");
  fill_common(p);
  p.A = static_cast<const uint16_t*>(a->A_full);
  p.B = static_cast<const uint16_t*>(a->B);
  p.C = static_cast<uint16_t*>(a->C);
  p.lda = a->K; p.ldb = a->N; p.ldc = a->N;
  p.M = (int)a->M; p.N = (int)a->N; p.K = (int)a->K;
  p.tiles_m = (int)(a->M / bm);
  p.tiles_n = (int)(a->N / 256);
  set_grid(p, total, n_prod, p.tiles_m * p.tiles_n);
  p.epoch = a->epoch;
  p.epoch_ptr = a->epoch_ptr;
  p.spin_limit = a->spin_limit;
  p.err = a->error_word;
  if (a->gated) {
    p.a_flags = a->flags;
    p.a_stage_order = a->stage_order;
    p.perm_mode = a->stage_order ? mk::kPermArrival : mk::kPermNone;
    if (n_prod > 0 || coop) {
      p.st_src = static_cast<const uint16_t*>(a->A_shards);
      p.st_dst = static_cast<uint16_t*>(a->A_full);
      p.st_cols = (int)a->K;
      p.st_nblocks = (int)nflags;
      p.st_order = a->stage_order;
      p.st_present = a->n_present;
      p.st_flags = a->flags;
      p.st_counters = a->stage_counters;
      // -1: halves alternate windows; -2: even share; <= -3: claimed
      p.st_coop = costage_waves ? 3 : coop ? (a->num_producers == -2 ? 1 : 2) : 0;
      p.st_batch = 8;
      if (costage_waves)
        p.st_claim = reinterpret_cast<uint32_t*>(static_cast<char*>(a->split_ws) + kClaimOffset);
    }
  }
  if (int rc = check_ws(a->split_ws, a->split_ws_bytes, "mk_ag_gemm")) return rc;
  plan_split(p, bm, a->split_ws, a->split_ws_bytes);
  *costage_out = costage_waves * total;
  return MK_OK;
}

int launch_ag(const mk::GemmKParams& p, int costage, void* stream) {
  hipError_t e = costage ? mk::launch_gemm_costaged(p, mk::kEpiStore, costage, static_cast<hipStream_t>(stream))
                         : mk::launch_gemm(p, 256, mk::kEpiStore, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_ag_gemm launch");
}
}  // namespace

extern "C" {

int mk_ag_gemm(const mk_ag_gemm_args* a, void* stream) {
  mk::GemmKParams p;
  int costage = 0;
  if (int rc = prepare_ag(a, stream, p, &costage)) return rc;
  return launch_ag(p, costage, stream);
}


int mk_ag_gemm_noalloc(const mk_ag_gemm_args* a, void* stream) {
  if (!a || !a->A_full || !a->B || !a->C) return fail(MK_EINVAL, "mk_ag_gemm_noalloc: null argument");
  if (a->split_ws || a->split_ws_bytes || a->stage_counters)
    return fail(MK_EINVAL, "mk_ag_gemm_noalloc: split_ws and stage_counters come from the library's static scratch; "
                           "pass them as NULL / 0");
  if (a->M < 0 || a->M / 128 > kNoAllocCounters)
    return fail(MK_ESHAPE, "mk_ag_gemm_noalloc: M=%lld exceeds the static scratch (at most %lld 128-row blocks)",
                (long long)a->M, (long long)kNoAllocCounters);
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  void* base = nullptr;
  if (int rc = scratch_ptr(&base)) return rc;
  mk_ag_gemm_args b = *a;
  b.split_ws = base;
  b.split_ws_bytes = kNoAllocSplitBytes;  // a tail split needing more partial tiles is not made
  b.stage_counters = reinterpret_cast<uint32_t*>(static_cast<char*>(base) + kNoAllocSplitBytes);
  // the co-resident staging kernel would need a side stream and events,
  // which the library creates on first use: stage cooperatively instead
  if (b.num_producers <= -3) b.num_producers = -1;
  // every argument check before anything is queued on the stream
  mk::GemmKParams p;
  int costage = 0;
  if (int rc = prepare_ag(&b, stream, p, &costage)) return rc;
  const int n_counters = (int)(a->M / 128);
  const int n_flags = (int)(kSplitFlagBytes / 4);
  const int n = std::max(n_flags, n_counters);
  hipLaunchKernelGGL(clear_scratch_kernel, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint32_t*>(base), n_flags, b.stage_counters, n_counters);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "mk_ag_gemm_noalloc scratch clear");
  return launch_ag(p, costage, stream);
}

int64_t mk_ag_gemm_noalloc_scratch_bytes(void) { return kNoAllocBytes; }

}  // extern "C"

namespace {
// GEMM + reduce-scatter epilogue; with peer_reduced also the all-gather half
// of a two-shot all-reduce (the other slices' reduced rows staged into
// `output`'s full matrix, done_flags per finished own tile).  `fn` names the
// entry point in errors.
int rs_launch(const mk_gemm_rs_args* a, const void* peer_reduced, uint16_t* full_out, uint32_t* done_flags,
              void* stream, const char* fn) {
  if (!a || !a->A || !a->B || !a->workspace || !a->output) return fail(MK_EINVAL, "%s: null argument", fn);
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  const int bm = 256;
  if (int rc = check_gemm_shape(a->M, a->N, a->K, bm)) return rc;
  if (a->world < 1 || a->rank < 0 || a->rank >= a->world) return fail(MK_EINVAL, "%s: bad world/rank", fn);
  if (a->M % a->world || (a->M / a->world) % bm)
    return fail(MK_ESHAPE, "%s: M/world must be a multiple of %d", fn, bm);
  if (a->M / bm > mk::kMaxTilesM) return fail(MK_ESHAPE, "%s: at most %d row tiles", fn, mk::kMaxTilesM);
  const int npeers = a->world - 1;
  if (npeers > 0 && !a->peer_recv) return fail(MK_EINVAL, "%s: peer_recv is null", fn);
  const int own_rows = (int)(a->M / a->world);
  int total;
  if (int rc = grid_total(a->num_cus, d, fn, &total)) return rc;
  if (a->num_producers < -6) return fail(MK_EINVAL, "%s: num_producers must be >= -6", fn);
  const bool coop = a->gated && npeers > 0 && a->num_producers < 0;
  int costage_waves = 0;
  if (int rc = costage_request(a->gated && npeers > 0, a->num_producers, a->split_ws, a->split_ws_bytes, stream, fn,
                               &costage_waves))
    return rc;
  const int n_prod = (a->gated && npeers > 0 && a->num_producers > 0) ? a->num_producers : 0;
  if (a->gated && npeers > 0) {
    if (!a->flags) return fail(MK_EINVAL, "%s: gated launch needs flags", fn);
    if (a->epoch == 0 && !a->epoch_ptr) return fail(MK_EINVAL, "%s: epoch 0 is reserved", fn);
    if (a->num_producers != 0 && !a->peer_src) return fail(MK_EINVAL, "%s: staging needs peer_src", fn);
    if (coop && !a->stage_counters) return fail(MK_EINVAL, "%s: cooperative staging needs stage_counters", fn);
  }
  if (n_prod >= total) return fail(MK_EINVAL, "%s: bad num_producers", fn);
  mk::GemmKParams p;
  fill_common(p);
  p.A = static_cast<const uint16_t*>(a->A);
  p.B = static_cast<const uint16_t*>(a->B);
  p.C = static_cast<uint16_t*>(a->workspace);
  p.lda = a->K; p.ldb = a->N; p.ldc = a->N;
  p.M = (int)a->M; p.N = (int)a->N; p.K = (int)a->K;
  p.tiles_m = (int)(a->M / bm);
  p.tiles_n = (int)(a->N / 256);
  set_grid(p, total, n_prod, p.tiles_m * p.tiles_n);
  // Owned row tiles spread one per round, in the order their peer blocks
  // arrive when this launch stages them.
  p.perm_mode = mk::kPermOwnedSpread;
  p.rs_own_row0 = a->rank * own_rows;
  p.rs_own_rows = own_rows;
  p.rs_npeers = npeers;
  p.rs_recv = static_cast<const uint16_t*>(a->peer_recv);
  p.rs_out = static_cast<uint16_t*>(a->output);
  p.ar_done = done_flags;
  p.epoch = a->epoch;
  p.epoch_ptr = a->epoch_ptr;
  p.spin_limit = a->spin_limit;
  p.err = a->error_word;
  if (a->gated && npeers > 0) {
    p.rs_flags = a->flags;
    if (n_prod > 0 || coop) {
      p.st_src = static_cast<const uint16_t*>(a->peer_src);
      p.st_dst = static_cast<uint16_t*>(a->peer_recv);
      p.st_cols = (int)a->N;
      p.st_nblocks = npeers * (own_rows / 128);
      if (peer_reduced) {
        // all-gather half: the peers' reduced slices, in slice order
        // without this rank's, into full_out around this rank's slice
        p.st_src2 = static_cast<const uint16_t*>(peer_reduced);
        p.st_dst2 = full_out;
        p.st_split_at = p.st_nblocks;
        p.st_dst2_skip_at = a->rank * (own_rows / 128);
        p.st_dst2_skip = own_rows / 128;
        p.st_nblocks *= 2;
      }
      p.st_order = a->stage_order;
      p.st_flags = a->flags;
      p.st_counters = a->stage_counters;
      // even share (measured faster here than alternating halves); <= -3: claimed
      p.st_coop = costage_waves ? 3 : coop ? 1 : 0;
      p.st_batch = 8;
      if (costage_waves)
        p.st_claim = reinterpret_cast<uint32_t*>(static_cast<char*>(a->split_ws) + kClaimOffset);
    }
  }
  if (int rc = check_ws(a->split_ws, a->split_ws_bytes, fn)) return rc;
  plan_split(p, bm, a->split_ws, a->split_ws_bytes);
  hipError_t e = costage_waves ? mk::launch_gemm_costaged(p, mk::kEpiReduce, costage_waves * total,
                                                          static_cast<hipStream_t>(stream))
                               : mk::launch_gemm(p, bm, mk::kEpiReduce, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, fn);
}
}  // namespace

extern "C" {

int mk_gemm_rs(const mk_gemm_rs_args* a, void* stream) {
  return rs_launch(a, nullptr, nullptr, nullptr, stream, "mk_gemm_rs");
}

int mk_gemm_ar_two_shot(const mk_gemm_ar2_args* a, void* stream) {
  if (!a || !a->C_final) return fail(MK_EINVAL, "mk_gemm_ar_two_shot: null argument");
  if (a->world < 1 || a->rank < 0 || a->rank >= a->world || a->M % a->world)
    return fail(MK_EINVAL, "mk_gemm_ar_two_shot: bad world/rank");
  const bool staging = a->gated && a->world > 1 && a->num_producers != 0;
  if (staging && !a->peer_reduced) return fail(MK_EINVAL, "mk_gemm_ar_two_shot: staging needs peer_reduced");
  if (a->done_flags && a->epoch == 0 && !a->epoch_ptr)
    return fail(MK_EINVAL, "mk_gemm_ar_two_shot: epoch 0 is reserved");
  mk_gemm_rs_args r;
  std::memset(&r, 0, sizeof r);
  r.A = a->A; r.B = a->B;
  r.workspace = a->sends;
  r.output = static_cast<uint16_t*>(a->C_final) + (int64_t)a->rank * (a->M / a->world) * a->N;
  r.peer_src = a->peer_src; r.peer_recv = a->peer_recv;
  r.M = a->M; r.N = a->N; r.K = a->K;
  r.world = a->world; r.rank = a->rank;
  r.flags = a->flags; r.stage_order = a->stage_order; r.epoch = a->epoch; r.gated = a->gated;
  r.num_producers = a->num_producers; r.num_cus = a->num_cus; r.spin_limit = a->spin_limit;
  r.error_word = a->error_word; r.stage_counters = a->stage_counters;
  r.split_ws = a->split_ws; r.split_ws_bytes = a->split_ws_bytes; r.epoch_ptr = a->epoch_ptr;
  return rs_launch(&r, staging ? a->peer_reduced : nullptr, static_cast<uint16_t*>(a->C_final), a->done_flags,
                   stream, "mk_gemm_ar_two_shot");
}

int mk_gemm_ar(const mk_gemm_ar_args* a, void* stream) {
  if (!a || !a->A || !a->B || !a->C_final) return fail(MK_EINVAL, "mk_gemm_ar: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  const int bm = 256;
  if (int rc = check_gemm_shape(a->M, a->N, a->K, bm)) return rc;
  if (a->world < 1) return fail(MK_EINVAL, "mk_gemm_ar: world must be >= 1");
  if (a->M / bm > mk::kMaxTilesM) return fail(MK_ESHAPE, "mk_gemm_ar: at most %d row tiles", mk::kMaxTilesM);
  const int npeers = a->world - 1;
  if (npeers > 0 && !a->peer_recv) return fail(MK_EINVAL, "mk_gemm_ar: peer_recv is null");
  const int64_t nflags = (int64_t)npeers * (a->M / 128);
  if (a->stage_order && nflags + a->M / bm > 8192)
    return fail(MK_ESHAPE, "mk_gemm_ar: too many flags for the arrival-order schedule");
  int total;
  if (int rc = grid_total(a->num_cus, d, "mk_gemm_ar", &total)) return rc;
  if (a->num_producers < -6) return fail(MK_EINVAL, "mk_gemm_ar: num_producers must be >= -6");
  const bool gated = a->gated && npeers > 0;
  const bool coop = gated && a->num_producers < 0;
  int costage_waves = 0;
  if (int rc = costage_request(gated, a->num_producers, a->split_ws, a->split_ws_bytes, stream, "mk_gemm_ar",
                               &costage_waves))
    return rc;
  const int n_prod = (gated && a->num_producers > 0) ? a->num_producers : 0;
  if (gated) {
    if (!a->flags) return fail(MK_EINVAL, "mk_gemm_ar: gated launch needs flags");
    if (a->num_producers != 0 && !a->peer_src) return fail(MK_EINVAL, "mk_gemm_ar: staging needs peer_src");
    if (coop && !a->stage_counters) return fail(MK_EINVAL, "mk_gemm_ar: cooperative staging needs stage_counters");
  }
  if ((gated || a->done_flags) && a->epoch == 0 && !a->epoch_ptr)
    return fail(MK_EINVAL, "mk_gemm_ar: epoch 0 is reserved");
  if (n_prod >= total) return fail(MK_EINVAL, "mk_gemm_ar: bad num_producers");
  mk::GemmKParams p;
  fill_common(p);
  p.A = static_cast<const uint16_t*>(a->A);
  p.B = static_cast<const uint16_t*>(a->B);
  p.C = static_cast<uint16_t*>(a->C_final);  // every row is owned: rs_out
  p.lda = a->K; p.ldb = a->N; p.ldc = a->N;
  p.M = (int)a->M; p.N = (int)a->N; p.K = (int)a->K;
  p.tiles_m = (int)(a->M / bm);
  p.tiles_n = (int)(a->N / 256);
  set_grid(p, total, n_prod, p.tiles_m * p.tiles_n);
  p.rs_own_row0 = 0;
  p.rs_own_rows = (int)a->M;
  p.rs_npeers = npeers;
  p.rs_recv = static_cast<const uint16_t*>(a->peer_recv);
  p.rs_out = static_cast<uint16_t*>(a->C_final);
  p.ar_done = a->done_flags;
  p.epoch = a->epoch;
  p.epoch_ptr = a->epoch_ptr;
  p.spin_limit = a->spin_limit;
  p.err = a->error_word;
  if (gated) {
    p.rs_flags = a->flags;
    if (a->stage_order) {
      p.perm_mode = mk::kPermPeerArrival;
      p.a_stage_order = a->stage_order;
    }
    if (n_prod > 0 || coop) {
      p.st_src = static_cast<const uint16_t*>(a->peer_src);
      p.st_dst = static_cast<uint16_t*>(a->peer_recv);
      p.st_cols = (int)a->N;
      p.st_nblocks = (int)nflags;
      p.st_order = a->stage_order;
      p.st_flags = a->flags;
      p.st_counters = a->stage_counters;
      // even share (measured faster here than alternating halves); <= -3: claimed
      p.st_coop = costage_waves ? 3 : coop ? 1 : 0;
      p.st_batch = 8;
      if (costage_waves)
        p.st_claim = reinterpret_cast<uint32_t*>(static_cast<char*>(a->split_ws) + kClaimOffset);
    }
  }
  if (int rc = check_ws(a->split_ws, a->split_ws_bytes, "mk_gemm_ar")) return rc;
  plan_split(p, bm, a->split_ws, a->split_ws_bytes);
  hipError_t e = costage_waves ? mk::launch_gemm_costaged(p, mk::kEpiReduce, costage_waves * total,
                                                          static_cast<hipStream_t>(stream))
                               : mk::launch_gemm(p, bm, mk::kEpiReduce, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_gemm_ar launch");
}

// ---------------------------------------------------------------------------
// MoE
// ---------------------------------------------------------------------------

int mk_moe_index_sizes(const int32_t* topk_ids, int32_t T, int32_t topk, int32_t e0, int32_t n_local,
                       int32_t row_block, int64_t* R_out, int64_t* R_pad_out) {
  if (!topk_ids || !R_out || !R_pad_out) return fail(MK_EINVAL, "mk_moe_index_sizes: null argument");
  if (T < 0 || topk <= 0 || n_local <= 0 || row_block <= 0 || e0 < 0)
    return fail(MK_EINVAL, "mk_moe_index_sizes: bad sizes");
  std::vector<int64_t> cnt(n_local, 0);
  for (int64_t i = 0; i < (int64_t)T * topk; ++i) {
    const int e = topk_ids[i] - e0;
    if (e >= 0 && e < n_local) ++cnt[e];
  }
  int64_t R = 0, Rp = 0;
  for (int e = 0; e < n_local; ++e) {
    R += cnt[e];
    Rp += (cnt[e] + row_block - 1) / row_block * row_block;
  }
  *R_out = R;
  *R_pad_out = Rp;
  return MK_OK;
}

int mk_moe_build_indices(const int32_t* topk_ids, const float* gates, int32_t T, int32_t topk, int32_t e0,
                         int32_t n_local, int32_t row_block, const mk_moe_index* o) {
  if (!topk_ids || !gates || !o) return fail(MK_EINVAL, "mk_moe_build_indices: null argument");
  int64_t R, Rp;
  if (int rc = mk_moe_index_sizes(topk_ids, T, topk, e0, n_local, row_block, &R, &Rp)) return rc;
  // expert_to_tokens: (token, k) pairs per local expert in ascending token
  // order (reference bench/dispatch_gemm_bench.py:153-160).
  std::vector<std::vector<std::pair<int32_t, int32_t>>> e2t(n_local);
  for (int32_t t = 0; t < T; ++t)
    for (int32_t k = 0; k < topk; ++k) {
      const int e = topk_ids[(int64_t)t * topk + k] - e0;
      if (e >= 0 && e < n_local) e2t[e].push_back({t, k});
    }
  std::vector<int32_t> owner_count(T, 0);
  int64_t r = 0;
  for (int e = 0; e < n_local; ++e) {
    const int64_t cnt = (int64_t)e2t[e].size();
    const int64_t padded = (cnt + row_block - 1) / row_block * row_block;
    if (o->padded_tokens_per_expert) o->padded_tokens_per_expert[e] = (int32_t)padded;
    if (o->local_rb_per_expert) o->local_rb_per_expert[e] = (int32_t)(cnt / row_block);
    for (int64_t i = 0; i < padded; ++i, ++r) {
      const bool real = i < cnt;
      const int32_t t = real ? e2t[e][i].first : -1;
      if (o->pull_indices) {
        o->pull_indices[3 * r + 0] = real ? 0 : -1;
        o->pull_indices[3 * r + 1] = real ? 0 : -1;
        o->pull_indices[3 * r + 2] = t;
      }
      if (o->row_expert) o->row_expert[r] = e;
      if (o->rb_expert && (r % row_block) == 0) o->rb_expert[r / row_block] = e;
      if (o->rb_rows) {
        if ((r % row_block) == 0) o->rb_rows[r / row_block] = 0;
        if (real) ++o->rb_rows[r / row_block];
      }
      if (o->row_weight) o->row_weight[r] = real ? gates[(int64_t)t * topk + e2t[e][i].second] : 0.f;
      if (real) ++owner_count[t];
    }
  }
  // Gather CSR (reference bench/dispatch_gemm_glu_combine_bench.py:222-293
  // with one producer GPU owning every token): slots are handed out in row
  // order, so token t's contributions occupy owner_offset[t] + 0, 1, ...
  std::vector<int32_t> off(T + 1, 0);
  for (int32_t t = 0; t < T; ++t) off[t + 1] = off[t] + owner_count[t];
  if (o->owner_offset) std::memcpy(o->owner_offset, off.data(), sizeof(int32_t) * (T + 1));
  std::vector<int32_t> running(T, 0);
  r = 0;
  for (int e = 0; e < n_local; ++e) {
    const int64_t cnt = (int64_t)e2t[e].size();
    const int64_t padded = (cnt + row_block - 1) / row_block * row_block;
    for (int64_t i = 0; i < padded; ++i, ++r) {
      if (i < cnt) {
        const int32_t t = e2t[e][i].first;
        const int32_t slot = off[t] + running[t]++;
        if (o->row_to_slot) o->row_to_slot[r] = slot;
        if (o->row_to_owner) o->row_to_owner[r] = 0;
        if (o->slot_to_row) o->slot_to_row[slot] = (int32_t)r;
      } else {
        if (o->row_to_slot) o->row_to_slot[r] = 0;
        if (o->row_to_owner) o->row_to_owner[r] = -1;
      }
    }
  }
  return MK_OK;
}

int mk_moe_permute(const mk_moe_permute_args* a, void* stream) {
  if (!a) return fail(MK_EINVAL, "mk_moe_permute: null argument");
  if (a->H <= 0 || a->H % 8) return fail(MK_ESHAPE, "mk_moe_permute: H must be a positive multiple of 8");
  if (a->R_pad < 0 || a->tokens_per_src <= 0 || a->devs_per_node <= 0) return fail(MK_EINVAL, "mk_moe_permute: bad sizes");
  if (a->R_pad == 0) return MK_OK;  // no routed rows: nothing to copy
  if (!a->tokens || !a->pull_indices || !a->post_tokens) return fail(MK_EINVAL, "mk_moe_permute: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  mk::PermuteKParams p{static_cast<const uint16_t*>(a->tokens), a->pull_indices,
                       static_cast<uint16_t*>(a->post_tokens), a->R_pad, a->H, a->n_src_rows,
                       a->tokens_per_src, a->devs_per_node, a->sizes ? a->sizes + 1 : nullptr};
  hipError_t e = mk::launch_permute(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_moe_permute launch");
}

static int grouped_gemm_impl(const void* A, const void* W, void* out, const int32_t* rb_expert,
                             const int32_t* expert_rows, const int32_t* rb_rows, int64_t R_pad, int64_t K,
                             int64_t Nw, int32_t E, int32_t mode, int32_t num_cus, void* split_ws,
                             int64_t split_ws_bytes, const int32_t* gather_pull, int64_t n_src_rows,
                             int32_t tokens_per_src, int32_t devs_per_node, int32_t tile_n,
                             const int64_t* sizes, hipStream_t stream) {
  if (tile_n != 0 && tile_n != 256 && tile_n != 512)
    return fail(MK_EINVAL, "mk_moe_grouped_gemm: tile_n must be 0, 256 or 512");
  if (tile_n == 512 && Nw % 512) return fail(MK_ESHAPE, "mk_moe_grouped_gemm: tile_n 512 needs Nw %% 512 == 0");
  if (mode != 0 && mode != 1) return fail(MK_EINVAL, "mk_moe_grouped_gemm: mode must be 0 or 1");
  if (E <= 0) return fail(MK_EINVAL, "mk_moe_grouped_gemm: num_experts must be positive");
  if (R_pad < 0) return fail(MK_ESHAPE, "mk_moe_grouped_gemm: R_pad < 0");
  if (R_pad == 0) return MK_OK;  // no routed rows
  if (!A || !W || !out || (!rb_expert && !expert_rows)) return fail(MK_EINVAL, "mk_moe_grouped_gemm: null argument");
  if (int rc = check_gemm_shape(R_pad, Nw, K, 128)) return rc;
  if (gather_pull && (n_src_rows <= 0 || tokens_per_src <= 0 || devs_per_node <= 0 ||
                      n_src_rows * K * 2 >= (1LL << 31)))
    return fail(MK_EINVAL, "mk_moe_grouped_gemm: fused dispatch needs n_src_rows, tokens_per_src, devs_per_node "
                           "> 0 and a token buffer below 2 GiB");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  mk::GemmKParams p;
  fill_common(p);
  p.A = static_cast<const uint16_t*>(A);
  p.B = static_cast<const uint16_t*>(W);
  p.C = static_cast<uint16_t*>(out);
  p.lda = K; p.ldb = Nw; p.ldc = mode == 1 ? Nw / 2 : Nw;
  p.b_expert_stride = K * Nw;
  p.M = (int)R_pad; p.N = (int)Nw; p.K = (int)K;
  // 128 x 512 tiles stream each expert's activation rows half as often per
  // weight byte as 128 x 256 tiles.
  const int bn = tile_n ? tile_n : (Nw % 512 == 0 ? 512 : 256);
  p.tiles_m = (int)(R_pad / 128);
  p.tiles_n = (int)(Nw / bn);
  p.rb_expert = rb_expert;
  p.expert_rows = expert_rows;
  p.rb_rows = rb_rows;
  p.n_experts = E;
  p.swiglu_I = (int)(Nw / 2);
  p.gather_pull = gather_pull;
  p.gather_rows = n_src_rows;
  p.gather_tps = tokens_per_src;
  p.gather_devs = devs_per_node;
  int total;
  if (int rc = grid_total(num_cus, d, "mk_moe_grouped_gemm", &total)) return rc;
  set_grid(p, total, 0, p.tiles_m * p.tiles_n);
  // Few column tiles (GEMM1: 2I / 512 = 8): walk all row blocks of one
  // weight column slice together, so an expert's row blocks share its weight
  // fetch in one XCD's L2 (measured 15 us faster on config 5's GEMM1, and
  // 6 us slower on GEMM2's 14 column tiles, which keeps groups of 8).
  if (p.tiles_n <= 8) p.group_m = p.tiles_m;
  // More column tiles without an epilogue (GEMM2: 7168 / 512 = 14): each
  // expert's tiles together, column-major inside its run of row tiles
  // (config-5 GEMM2 210.9 -> 203.7 us; GEMM1 + SwiGLU measured 6 us slower
  // with it and keeps the order above).
  if (p.tiles_n > 8 && mode == 0 && rb_expert) p.expert_order = 1;
  // The grouped GEMMs are bound by the chip's weight streaming.  When the
  // tail round cannot be K-split (more tail tiles than half the grid),
  // every workgroup runs the same number of whole-tile rounds either way;
  // spreading the tiles evenly over ceil(tiles / rounds) workgroups (a
  // multiple of 8, for the XCD remap) gives each of them more bandwidth:
  // config-5 GEMM2 (658 tiles) 244 -> 231 us on 224 instead of 256.
  if (!sizes) {
    const int ntiles = p.tiles_m * p.tiles_n, R = ntiles % p.n_cons;
    if (num_cus <= 0 && R != 0 && 2 * R > p.n_cons) {
      const int rounds = (ntiles + p.n_cons - 1) / p.n_cons;
      const int even = ((ntiles + rounds - 1) / rounds + 7) / 8 * 8;
      if (even < p.n_cons) set_grid(p, even, 0, ntiles);
    }
  }
  if (int rc = check_ws(split_ws, split_ws_bytes, "mk_moe_grouped_gemm")) return rc;
  if (sizes) {
    // Row count on the device: the kernel clamps its row tiles to it and
    // plans the tail split itself, which may use up to one partial tile per
    // consumer (and one flag word each).
    p.rows_dev = sizes + 1;
    p.spread_dev = num_cus <= 0 ? 1 : 0;  // the library's grid: the kernel applies the tail spread
    if (split_ws && p.waves == 8 && (int64_t)p.n_cons * 4 <= kClaimOffset &&
        split_ws_bytes >= kSplitFlagBytes + (int64_t)p.n_cons * 128 * bn * 4) {
      p.sk_dev = 1;
      p.sk_flags = static_cast<uint32_t*>(split_ws);
      p.sk_ws = reinterpret_cast<float*>(static_cast<char*>(split_ws) + kSplitFlagBytes);
    }
  } else {
    plan_split(p, 128, split_ws, split_ws_bytes, bn);
  }
  hipError_t e = mk::launch_gemm(p, 128, mode == 1 ? mk::kEpiSwiGLU : mk::kEpiStore, stream, bn);
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_moe_grouped_gemm launch");
}

int mk_moe_grouped_gemm(const mk_moe_grouped_gemm_args* a, void* stream) {
  if (!a) return fail(MK_EINVAL, "mk_moe_grouped_gemm: null argument");
  return grouped_gemm_impl(a->A, a->W, a->out, a->rb_expert, a->padded_tokens_per_expert, a->rb_rows, a->R_pad, a->K, a->Nw, a->num_experts, a->mode,
                           a->num_cus, a->split_ws, a->split_ws_bytes, a->gather_pull, a->n_src_rows,
                           a->tokens_per_src, a->devs_per_node, a->tile_n, a->sizes,
                           static_cast<hipStream_t>(stream));
}

int mk_moe_combine(const mk_moe_combine_args* a, void* stream) {
  // y_expert, row_weight and slot_to_row are read only inside owner_offset's
  // ranges: with no routed rows (every range empty) they may be NULL.
  if (!a || !a->owner_offset || (!a->y_out && a->num_tokens > 0))
    return fail(MK_EINVAL, "mk_moe_combine: null argument");
  if (a->num_tokens < 0) return fail(MK_ESHAPE, "mk_moe_combine: num_tokens < 0");
  if (a->H <= 0 || a->H % 8) return fail(MK_ESHAPE, "mk_moe_combine: H must be a positive multiple of 8");
  if (a->out_dtype != 0 && a->out_dtype != 1) return fail(MK_EINVAL, "mk_moe_combine: out_dtype must be 0 or 1");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  mk::CombineKParams p{static_cast<const uint16_t*>(a->y_expert), a->row_weight, a->owner_offset, a->slot_to_row,
                       a->y_out, a->num_tokens, a->H, a->out_dtype};
  hipError_t e = mk::launch_combine(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_moe_combine launch");
}

int mk_moe_invert_slots(const int32_t* row_to_slot, const int32_t* row_to_owner, int64_t R_pad, int32_t owner,
                        int64_t slot_capacity, int32_t* slot_to_row, uint32_t* error_word, void* stream) {
  if (R_pad < 0 || slot_capacity < 0) return fail(MK_EINVAL, "mk_moe_invert_slots: R_pad and slot_capacity must be >= 0");
  if (slot_capacity > (1LL << 31)) return fail(MK_ESHAPE, "mk_moe_invert_slots: slot_capacity above 2^31");
  if (owner < 0) return fail(MK_EINVAL, "mk_moe_invert_slots: owner must be >= 0");
  if (R_pad == 0 && slot_capacity == 0) return MK_OK;
  if ((R_pad > 0 && (!row_to_slot || !row_to_owner)) || (slot_capacity > 0 && !slot_to_row))
    return fail(MK_EINVAL, "mk_moe_invert_slots: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  hipError_t e = mk::launch_invert_slots(row_to_slot, row_to_owner, R_pad, owner, slot_capacity, slot_to_row,
                                         error_word, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_moe_invert_slots launch");
}

int mk_moe_tile_rows(const int32_t* pull_indices, int64_t R_pad, int32_t* rb_rows, void* stream) {
  if (R_pad < 0 || R_pad % 128) return fail(MK_ESHAPE, "mk_moe_tile_rows: R_pad must be a multiple of 128");
  if (R_pad == 0) return MK_OK;
  if (!pull_indices || !rb_rows) return fail(MK_EINVAL, "mk_moe_tile_rows: null argument");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  hipError_t e = mk::launch_tile_rows(pull_indices, R_pad, rb_rows, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_moe_tile_rows launch");
}

int64_t mk_moe_index_workspace_bytes(int32_t num_tokens, int32_t topk, int32_t n_local) {
  if (num_tokens < 0 || topk <= 0 || n_local <= 0) return -1;
  return mk::index_workspace_bytes(num_tokens, topk, n_local);
}

int mk_moe_build_indices_dev(const mk_moe_index_dev_args* a, void* stream) {
  if (!a || !a->topk_ids || !a->topk_gates || !a->sizes) return fail(MK_EINVAL, "mk_moe_build_indices_dev: null argument");
  if (a->num_tokens < 0 || a->topk <= 0 || a->n_local <= 0 || a->row_block <= 0 || a->expert_begin < 0)
    return fail(MK_EINVAL, "mk_moe_build_indices_dev: bad sizes");
  if ((int64_t)a->num_tokens * a->topk + (int64_t)a->n_local * a->row_block > (1LL << 31))
    return fail(MK_ESHAPE, "mk_moe_build_indices_dev: too many rows for 32-bit row indices");
  if (a->capacity_rows < 0) return fail(MK_EINVAL, "mk_moe_build_indices_dev: capacity_rows < 0");
  if (a->n_local > 4096)
    return fail(MK_ESHAPE, "mk_moe_build_indices_dev: at most 4096 local experts (per-wave expert counts live in LDS)");
  if (!a->workspace || a->workspace_bytes < mk::index_workspace_bytes(a->num_tokens, a->topk, a->n_local))
    return fail(MK_EINVAL, "mk_moe_build_indices_dev: workspace smaller than mk_moe_index_workspace_bytes");
  DevInfo d;
  if (int rc = device_info(&d)) return rc;
  hipError_t e = mk::launch_build_indices(a->topk_ids, a->topk_gates, a->num_tokens, a->topk, a->expert_begin,
                                          a->n_local, a->row_block, a->capacity_rows, a->workspace, a->sizes,
                                          a->out, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MK_OK : hip_fail(e, "mk_moe_build_indices_dev launch");
}

int mk_moe_ffn_combine(const mk_moe_ffn_args* a, void* stream) {
  if (!a) return fail(MK_EINVAL, "mk_moe_ffn_combine: null argument");
  // every buffer the sequence touches, before anything is queued (buffers
  // of no rows may be NULL)
  const bool rows = a->R_pad > 0;
  if ((rows && (!a->tokens || !a->pull_indices || !a->w1 || !a->w2 || !a->act || !a->y_expert || !a->row_weight ||
                !a->slot_to_row || (!a->rb_expert && !a->padded_tokens_per_expert) ||
                (!a->fuse_dispatch && !a->post_tokens))) ||
      (a->num_tokens > 0 && (!a->owner_offset || !a->y_out)))
    return fail(MK_EINVAL, "mk_moe_ffn_combine: null argument");
  if (a->I % 128) return fail(MK_ESHAPE, "mk_moe_ffn_combine: I must be a multiple of 128");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->fuse_dispatch) {
    if (!a->pull_indices && a->R_pad > 0) return fail(MK_EINVAL, "mk_moe_ffn_combine: null argument");
    if (int rc = grouped_gemm_impl(a->tokens, a->w1, a->act, a->rb_expert, a->padded_tokens_per_expert, a->rb_rows,
                                   a->R_pad, a->H, 2 * a->I, a->num_experts, 1, a->num_cus, a->split_ws,
                                   a->split_ws_bytes, a->pull_indices, a->n_src_rows, a->tokens_per_src,
                                   a->devs_per_node, a->tile_n, a->sizes, s))
      return rc;
  } else {
    mk_moe_permute_args pa{a->tokens, a->pull_indices, a->post_tokens, a->R_pad, a->H,
                           a->n_src_rows, a->tokens_per_src, a->devs_per_node, a->sizes};
    if (int rc = mk_moe_permute(&pa, stream)) return rc;
    if (int rc = grouped_gemm_impl(a->post_tokens, a->w1, a->act, a->rb_expert, a->padded_tokens_per_expert,
                                   a->rb_rows, a->R_pad, a->H, 2 * a->I, a->num_experts, 1, a->num_cus,
                                   a->split_ws, a->split_ws_bytes, nullptr, 0, 0, 0, a->tile_n, a->sizes, s))
      return rc;
  }
  if (int rc = grouped_gemm_impl(a->act, a->w2, a->y_expert, a->rb_expert, a->padded_tokens_per_expert,
                                 a->rb_rows, a->R_pad, a->I, a->H, a->num_experts, 0, a->num_cus, a->split_ws,
                                 a->split_ws_bytes, nullptr, 0, 0, 0, a->tile_n, a->sizes, s))
    return rc;
  mk_moe_combine_args ca{a->y_expert, a->row_weight, a->owner_offset, a->slot_to_row, a->y_out,
                         a->num_tokens, a->H, a->out_dtype};
  return mk_moe_combine(&ca, stream);
}

}  // extern "C"
