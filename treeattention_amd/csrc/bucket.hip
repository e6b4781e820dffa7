// Bucketing of (query, distinct leaf block) pairs by leaf block, per
// (batch, head): a stable counting sort so each leaf block's pairs are one
// contiguous, deterministic run.  Every ancestor of a leaf block covers a
// contiguous range of blocks, so the same order groups pairs by tree node at
// every level.
//
// One wavefront scans a chunk of queries in position order; a query's
// distinct blocks are different lanes with different counters, so LDS
// counters give ranks that do not depend on scheduling.
#include "launch.h"

namespace ta {

constexpr int kWin = 8192;  // leaf-block counters held in LDS per pass

struct BucketArgs {
  int L, H, S, NL, qc, nchunk;
  const int* slot_leaf;
  const int* slot_count;
  int* hist;         // (BH, NL, nchunk)
  int* block_start;  // (BH, NL+1)
  int* order;        // (BH, L*S)
};

// grid (nchunk, BH), block 64.  kScatter=false: counts per (block, chunk);
// kScatter=true: writes order[] using the scanned hist as bases.
template <bool kScatter>
__global__ __launch_bounds__(64) void bucket_pass_kernel(BucketArgs a) {
  __shared__ int cnt[kWin];
  const int c = blockIdx.x, bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int lane = threadIdx.x;
  const int q0 = c * a.qc, q1 = min(a.L, q0 + a.qc);
  const int64_t LS = (int64_t)a.L * a.S;
  for (int w0 = 0; w0 < a.NL; w0 += kWin) {
    const int wn = min(kWin, a.NL - w0);
    for (int i = lane; i < wn; i += 64) cnt[i] = 0;
    __syncthreads();
    for (int l = q0; l < q1; ++l) {
      const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
      const int n = a.slot_count[qh];
      if (lane < n) {
        const int beta = a.slot_leaf[qh * a.S + lane] - w0;
        if (beta >= 0 && beta < wn) {
          const int r = atomicAdd(&cnt[beta], 1);
          if constexpr (kScatter) {
            const int base = a.hist[((int64_t)bh * a.NL + w0 + beta) * a.nchunk + c];
            a.order[(int64_t)bh * LS + base + r] = l * a.S + lane;
          }
        }
      }
      __syncthreads();
    }
    if constexpr (!kScatter) {
      for (int i = lane; i < wn; i += 64) a.hist[((int64_t)bh * a.NL + w0 + i) * a.nchunk + c] = cnt[i];
    }
    __syncthreads();
  }
}

// Exclusive scan of hist[bh] (block-major, chunk-minor) in place; one
// workgroup of 1024 threads per (batch, head).
__global__ __launch_bounds__(1024) void bucket_scan_kernel(BucketArgs a) {
  __shared__ int part[1024];
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int64_t n = (int64_t)a.NL * a.nchunk;
  int* hh = a.hist + (int64_t)bh * n;
  const int64_t per = (n + 1023) / 1024;
  const int64_t s0 = tid * per, s1 = min(n, s0 + per);
  int sum = 0;
  for (int64_t i = s0; i < s1; ++i) sum += hh[i];
  part[tid] = sum;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = part[tid] - sum;
  for (int64_t i = s0; i < s1; ++i) {
    const int x = hh[i];
    hh[i] = run;
    run += x;
  }
  __syncthreads();
  int* bs = a.block_start + (int64_t)bh * (a.NL + 1);
  for (int beta = tid; beta < a.NL; beta += 1024) bs[beta] = hh[(int64_t)beta * a.nchunk];
  if (tid == 1023) bs[a.NL] = part[1023];
}

hipError_t launch_bucket(const Plan& P, char* rec, hipStream_t st) {
  BucketArgs a;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.NL = P.geo.NL;
  a.qc = P.qc;
  a.nchunk = P.nchunk;
  a.slot_leaf = (const int*)(rec + P.rec.slot_leaf);
  a.slot_count = (const int*)(rec + P.rec.slot_count);
  a.hist = (int*)(rec + P.rec.hist);
  a.block_start = (int*)(rec + P.rec.block_start);
  a.order = (int*)(rec + P.rec.order);
  hipLaunchKernelGGL(bucket_pass_kernel<false>, dim3(P.nchunk, P.BH), dim3(64), 0, st, a);
  hipLaunchKernelGGL(bucket_scan_kernel, dim3(P.BH), dim3(1024), 0, st, a);
  hipLaunchKernelGGL(bucket_pass_kernel<true>, dim3(P.nchunk, P.BH), dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace ta
