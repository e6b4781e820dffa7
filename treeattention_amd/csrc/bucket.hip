// Bucketing of (query, distinct leaf block) pairs by leaf block, per
// (batch, head): a stable counting sort so each leaf block's pairs are one
// contiguous, deterministic run in query order.  Every ancestor of a leaf
// block covers a contiguous range of blocks, so the same order groups pairs
// by tree node at every level.
//
// A query lists each leaf block at most once, so within a chunk of
// kQueryChunk queries the rank of (query l, block beta) in beta's run is the
// number of earlier queries of the chunk that also picked beta: one bit per
// (block, query) in LDS and a popcount give it without any ordering between
// threads.
#include "launch.h"

namespace ta {

constexpr int kWin = 2048;                 // leaf blocks per LDS window
constexpr int kWords = kQueryChunk / 32;  // bitmask words per block

struct BucketArgs {
  int L, H, S, NL, nchunk, npiece, nseg;
  const int* slot_leaf;
  const int* slot_count;
  int* hist;         // (BH, NL, nchunk)
  int* block_start;  // (BH, NL+1)
  int* order;        // (BH, L*S)
  int* piece_start;  // (BH, NL+1)
  int* piece_block;  // (BH, npiece)
  int* seg_sum;      // (BH, nseg) large histograms: counts per scan segment
};

// grid (nchunk, BH), block kQueryChunk (one thread per query of the chunk).
template <bool kScatter>
__global__ __launch_bounds__(kQueryChunk) void bucket_pass_kernel(BucketArgs a) {
  __shared__ uint32_t bits[kWin * kWords];
  __shared__ int hb[kScatter ? kWin : 1];  // scatter: the window's run bases of this chunk
  const int c = blockIdx.x, bh = blockIdx.y, bb = bh / a.H, h = bh - bb * a.H;
  const int tid = threadIdx.x;
  const int l = c * kQueryChunk + tid;
  const bool act = l < a.L;
  const int64_t qh = ((int64_t)bb * a.L + l) * a.H + h;
  const int n = act ? a.slot_count[qh] : 0;
  const int* mine = a.slot_leaf + qh * a.S;
  const int64_t LS = (int64_t)a.L * a.S;
  const uint32_t bit = 1u << (tid & 31);
  const int word = tid >> 5;
  // fn(u, leaf) for this query's slots, eight slot loads in flight at a time
  auto for_slots = [&](auto fn) {
    for (int u0 = 0; u0 < n; u0 += 8) {
      int lv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) lv[j] = u0 + j < n ? mine[u0 + j] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (u0 + j < n) fn(u0 + j, lv[j]);
    }
  };
  for (int w0 = 0; w0 < a.NL; w0 += kWin) {
    const int wn = min(kWin, a.NL - w0);
    for (int i = tid; i < wn * kWords; i += kQueryChunk) bits[i] = 0u;
    if constexpr (kScatter)
      for (int beta = tid; beta < wn; beta += kQueryChunk) hb[beta] = a.hist[((int64_t)bh * a.NL + w0 + beta) * a.nchunk + c];
    __syncthreads();
    for_slots([&](int u, int leaf) {
      const int beta = leaf - w0;
      if (beta >= 0 && beta < wn) atomicOr(&bits[beta * kWords + word], bit);
    });
    __syncthreads();
    if constexpr (!kScatter) {
      for (int beta = tid; beta < wn; beta += kQueryChunk) {
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < kWords; ++k) cnt += __popc(bits[beta * kWords + k]);
        a.hist[((int64_t)bh * a.NL + w0 + beta) * a.nchunk + c] = cnt;
      }
    } else {
      for_slots([&](int u, int leaf) {
        const int beta = leaf - w0;
        if (beta < 0 || beta >= wn) return;
        const uint32_t* bm = bits + beta * kWords;
        int r = __popc(bm[word] & (bit - 1u));
        for (int k = 0; k < word; ++k) r += __popc(bm[k]);
        a.order[(int64_t)bh * LS + hb[beta] + r] = l * a.S + u;
      });
    }
    __syncthreads();
  }
}

constexpr int kScanBatch = 16;  // counts loaded per batch by one scan thread

// Exclusive prefix of v over the 1024 threads of the workgroup (and the
// total): a shuffle scan inside each wave, then over the 16 wave totals.
// part must hold 16 ints; every thread calls it.
__device__ __forceinline__ int block_scan_1024(int v, int* part, int tid, int& total) {
  const int lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();  // part[] is free (an earlier scan's readers are done)
  if (lane == 63) part[w] = x;
  __syncthreads();
  int base = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = part[i];
    if (i < w) base += t;
    total += t;
  }
  return base + x - v;
}

// The leaf-forward pieces from the block starts bs: block beta with n pairs
// gets ceil(n / kPieceFwd) pieces, numbered by an exclusive scan over beta,
// and piece_block names each piece's block (-1 past the last).  All 1024
// threads call it.
__device__ __forceinline__ void bucket_pieces(const BucketArgs& a, int bh, const int* bs, int* part, int tid) {
  const int perb = (a.NL + 1023) / 1024;
  const int b0 = min(a.NL, tid * perb), b1 = min(a.NL, b0 + perb);
  int np = 0;
  for (int beta = b0; beta < b1; ++beta) np += (bs[beta + 1] - bs[beta] + kPieceFwd - 1) / kPieceFwd;
  int* ps = a.piece_start + (int64_t)bh * (a.NL + 1);
  int* pb = a.piece_block + (int64_t)bh * a.npiece;
  int npt;
  int pr = block_scan_1024(np, part, tid, npt);
  for (int beta = b0; beta < b1; ++beta) {
    ps[beta] = pr;
    const int m = (bs[beta + 1] - bs[beta] + kPieceFwd - 1) / kPieceFwd;
    for (int j = 0; j < m; ++j) pb[pr + j] = beta;
    pr += m;
  }
  if (tid == 1023) ps[a.NL] = npt;
  for (int i = npt + tid; i < a.npiece; i += 1024) pb[i] = -1;
}

// Exclusive scan of hist[bh] (block-major, chunk-minor) in place, the block
// starts, then the leaf-forward pieces: block beta with n pairs gets
// ceil(n / kPieceFwd) pieces, numbered by an exclusive scan over beta, and
// piece_block names each piece's block (-1 past the last).  One workgroup of
// 1024 threads per (batch, head).
__global__ __launch_bounds__(1024) void bucket_scan_kernel(BucketArgs a) {
  __shared__ int part[1024];
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int64_t n = (int64_t)a.NL * a.nchunk;
  int* hh = a.hist + (int64_t)bh * n;
  const int64_t per = (n + 1023) / 1024;
  const int64_t s0 = tid * per, s1 = min(n, s0 + per);
  // each thread's run of counts, kScanBatch loads in flight at a time
  int sum = 0;
  for (int64_t i0 = s0; i0 < s1; i0 += kScanBatch) {
    int x[kScanBatch];
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) x[j] = i0 + j < s1 ? hh[i0 + j] : 0;
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) sum += x[j];
  }
  int total;
  int run = block_scan_1024(sum, part, tid, total);
  for (int64_t i0 = s0; i0 < s1; i0 += kScanBatch) {
    int x[kScanBatch];
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) x[j] = i0 + j < s1 ? hh[i0 + j] : 0;
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j)
      if (i0 + j < s1) {
        hh[i0 + j] = run;
        run += x[j];
      }
  }
  __syncthreads();
  int* bs = a.block_start + (int64_t)bh * (a.NL + 1);
  for (int beta = tid; beta < a.NL; beta += 1024) bs[beta] = hh[(int64_t)beta * a.nchunk];
  if (tid == 1023) bs[a.NL] = total;
  __syncthreads();  // block starts (global, this workgroup's writes) visible; part[] reused below

  bucket_pieces(a, bh, bs, part, tid);
}

// Large histograms (many leaf blocks x query chunks): the scan runs over
// segments of kSegScan counts, 16 per thread of a 1024-thread workgroup:
// bucket_segsum_kernel sums each segment, bucket_segscan_kernel adds the sums
// of the segments before its own and rescans it in place (writing the block
// starts that fall in it), bucket_pieces_kernel builds the piece table.
constexpr int kSegScan = 1024 * kScanBatch;

__global__ __launch_bounds__(1024) void bucket_segsum_kernel(BucketArgs a) {
  __shared__ int part[16];
  const int seg = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int64_t n = (int64_t)a.NL * a.nchunk;
  const int* hh = a.hist + (int64_t)bh * n;
  const int64_t s0 = (int64_t)seg * kSegScan + tid * kScanBatch;
  int x[kScanBatch], sum = 0;
#pragma unroll
  for (int j = 0; j < kScanBatch; ++j) x[j] = s0 + j < n ? hh[s0 + j] : 0;
#pragma unroll
  for (int j = 0; j < kScanBatch; ++j) sum += x[j];
  int total;
  block_scan_1024(sum, part, tid, total);
  if (tid == 0) a.seg_sum[(int64_t)bh * a.nseg + seg] = total;
}

__global__ __launch_bounds__(1024) void bucket_segscan_kernel(BucketArgs a) {
  __shared__ int part[16];
  __shared__ int offs;
  const int seg = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int64_t n = (int64_t)a.NL * a.nchunk;
  int* hh = a.hist + (int64_t)bh * n;
  const int* ss = a.seg_sum + (int64_t)bh * a.nseg;
  // the sums of the earlier segments
  int pre = 0;
  for (int i = tid; i < seg; i += 1024) pre += ss[i];
  int ptot;
  block_scan_1024(pre, part, tid, ptot);
  if (tid == 0) offs = ptot;
  const int64_t s0 = (int64_t)seg * kSegScan + tid * kScanBatch;
  int x[kScanBatch], sum = 0;
#pragma unroll
  for (int j = 0; j < kScanBatch; ++j) x[j] = s0 + j < n ? hh[s0 + j] : 0;
#pragma unroll
  for (int j = 0; j < kScanBatch; ++j) sum += x[j];
  int total;
  int run = block_scan_1024(sum, part, tid, total);  // its barriers also publish offs
  run += offs;
  int* bs = a.block_start + (int64_t)bh * (a.NL + 1);
#pragma unroll
  for (int j = 0; j < kScanBatch; ++j)
    if (s0 + j < n) {
      hh[s0 + j] = run;
      if ((s0 + j) % a.nchunk == 0) bs[(s0 + j) / a.nchunk] = run;
      run += x[j];
    }
  if (seg == a.nseg - 1 && tid == 1023) bs[a.NL] = offs + total;
}

__global__ __launch_bounds__(1024) void bucket_pieces_kernel(BucketArgs a) {
  __shared__ int part[16];
  const int bh = blockIdx.x;
  bucket_pieces(a, bh, a.block_start + (int64_t)bh * (a.NL + 1), part, threadIdx.x);
}

hipError_t launch_bucket(const Plan& P, char* rec, hipStream_t st) {
  BucketArgs a;
  a.L = (int)P.L;
  a.H = (int)P.H;
  a.S = (int)P.S;
  a.NL = P.geo.NL;
  a.nchunk = P.nchunk;
  a.slot_leaf = (const int*)(rec + P.rec.slot_leaf);
  a.slot_count = (const int*)(rec + P.rec.slot_count);
  a.hist = (int*)(rec + P.rec.hist);
  a.block_start = (int*)(rec + P.rec.block_start);
  a.order = (int*)(rec + P.rec.order);
  a.npiece = P.npiece;
  a.piece_start = (int*)(rec + P.rec.piece_start);
  a.piece_block = (int*)(rec + P.rec.piece_block);
  a.nseg = P.nseg;
  a.seg_sum = (int*)(rec + P.rec.seg_sum);
  hipLaunchKernelGGL(bucket_pass_kernel<false>, dim3(P.nchunk, P.BH), dim3(kQueryChunk), 0, st, a);
  if (P.nseg > 4) {
    hipLaunchKernelGGL(bucket_segsum_kernel, dim3(P.nseg, P.BH), dim3(1024), 0, st, a);
    hipLaunchKernelGGL(bucket_segscan_kernel, dim3(P.nseg, P.BH), dim3(1024), 0, st, a);
    hipLaunchKernelGGL(bucket_pieces_kernel, dim3(P.BH), dim3(1024), 0, st, a);
  } else {
    hipLaunchKernelGGL(bucket_scan_kernel, dim3(P.BH), dim3(1024), 0, st, a);
  }
  hipLaunchKernelGGL(bucket_pass_kernel<true>, dim3(P.nchunk, P.BH), dim3(kQueryChunk), 0, st, a);
  return hipGetLastError();
}

}  // namespace ta
