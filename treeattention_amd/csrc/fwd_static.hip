// ta_forward_static: the whole forward (ta_forward) for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The forward's only scratch -- the w * o
// row of every (query, distinct leaf block) pair that the combine sums -- lives
// in a file-scope device array instead of a caller workspace, and the leaf
// forward runs over groups of (batch, head)s whose rows fit in it (the same
// kernels as ta_forward, so the results are bit-identical).
#include <mutex>

#include "launch.h"

namespace ta {
namespace {

constexpr int64_t kScratchBytes = TA_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

// One copy per GPU; held by every device the library runs this entry point on
// until the process ends.  Host code never uses the name itself (it is a host
// stand-in, not a device address): only the per-device pointer below.
static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of this GPU's `scratch` (looked up once per device, with the
// device current).
int scratch_address(hipStream_t st, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return fail(TA_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  int dev = cur;
  if (st) {
    hipDevice_t sd = 0;
    e = hipStreamGetDevice(st, &sd);
    if (e != hipSuccess) return fail(TA_ERR_INVALID, "hipStreamGetDevice: %s", hipGetErrorString(e));
    dev = (int)sd;
  }
  if (dev != cur)
    return fail(TA_ERR_INVALID, "the stream belongs to device %d but device %d is current", dev, cur);
  if (dev < 0 || dev >= kMaxDevices) return fail(TA_ERR_UNSUPPORTED, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return TA_OK;
}

}  // namespace
}  // namespace ta

using namespace ta;

extern "C" int ta_forward_static(const ta_problem* p, const void* q, const void* k, const void* v,
                                 const float* uniforms, uint64_t seed, void* out, float* weights, void* record,
                                 void* stream) {
  Plan P;
  int rc = make_plan(p, &P);
  if (rc) return rc;
  // pair rows of one (batch, head) (none for one-token leaves: their leaf stage is a value gather)
  const int64_t per_bh = P.geo.LB == 1 ? 0 : P.L * P.S * P.D * P.esize;
  if (per_bh > kScratchBytes)
    return fail(TA_ERR_UNSUPPORTED,
                "ta_forward_static: one (batch, head)'s pair rows take %lld bytes (L*num_samples*head_dim*%d), "
                "more than its %lld-byte static scratch; use ta_forward with a workspace",
                (long long)per_bh, P.esize, (long long)kScratchBytes);
  const bool need_k = p->tree_mode != TA_TREE_NODEKEYS;
  if (!q || !v || !out || !weights || !record || (need_k && !k))
    return fail(TA_ERR_INVALID, "NULL device pointer");
  hipStream_t st = (hipStream_t)stream;
  void* scr = nullptr;
  rc = scratch_address(st, &scr);
  if (rc) return rc;
  rc = ta_pool(p, k, record, stream);
  if (rc) return rc;
  rc = ta_sample(p, q, uniforms, seed, weights, record, stream);
  if (rc) return rc;
  rc = ta_bucket(p, record, stream);
  if (rc) return rc;
  if (((uintptr_t)q | (uintptr_t)v | (uintptr_t)out | (uintptr_t)record | (need_k ? (uintptr_t)k : 0)) & 15)
    return fail(TA_ERR_INVALID, "q/k/v/out/record must be 16-byte aligned device pointers");
  const int group = (int)(per_bh == 0 || kScratchBytes / per_bh >= P.BH ? P.BH : kScratchBytes / per_bh);
  for (int bh0 = 0; bh0 < P.BH; bh0 += group) {
    const int nbh = (int)(P.BH - bh0 < group ? P.BH - bh0 : group);
    hipError_t e = launch_leaf_fwd_group(P, q, k, v, out, (char*)record, scr, bh0, nbh, st);
    if (e != hipSuccess) return fail(TA_ERR_LAUNCH, "leaf_forward: %s", hipGetErrorString(e));
  }
  return ok();
}
