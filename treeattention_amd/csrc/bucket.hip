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

constexpr int kWin = kBucketWin;           // leaf blocks per LDS window
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

// Many leaf blocks (more than one LDS window, e.g. the reference's one-token
// leaves): the (block x query chunk) table would grow as NL L; instead every
// slot becomes a key (batch * head) * (NL + 1) + leaf block (NL for the slots
// past a query's count) with value l * S + u, in (batch, position, head, slot)
// order, and a stable LSD radix sort orders them: within one (batch, head) and
// leaf block the values keep their (l, u) order -- exactly the counting sort's
// result -- and each (batch, head)'s L S entries, its pairs first, land in its
// own range of `order`.  The block starts are an exclusive scan of per-block
// counts.  Per 8-bit digit: per-tile digit counts, exclusive scans of the
// per-digit rows over tiles, then a scatter whose ranks within a tile come from wavefront
// ballots (peers with the same digit) and per-wave digit counts in LDS.  No
// atomics decide any order; no memset or library call (graph-capture safe).
constexpr int kSortTile = 2048;  // elements per workgroup: 8 rounds of 256

__global__ __launch_bounds__(256) void sort_keys_kernel(BucketArgs a, uint32_t* keys, int* vals, int* cnt,
                                                        int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t qh = i / a.S;
  const int u = (int)(i - qh * a.S);
  const int h = (int)(qh % a.H);
  const int64_t bl = qh / a.H;
  const int l = (int)(bl % a.L), bb = (int)(bl / a.L);
  const int64_t bh = (int64_t)bb * a.H + h;
  const bool act = u < a.slot_count[qh];
  const int leaf = act ? a.slot_leaf[i] : a.NL;
  keys[i] = (uint32_t)(bh * (a.NL + 1) + leaf);
  vals[i] = l * a.S + u;
  if (act) atomicAdd(cnt + bh * a.NL + leaf, 1);  // counts: order-free
}

__global__ __launch_bounds__(256) void zero_ints_kernel(int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// th[digit * ntiles + tile] = elements of the tile with that digit
__global__ __launch_bounds__(256) void radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                         int* __restrict__ th, int ntiles) {
  __shared__ int cnt[256];
  const int tile = blockIdx.x, tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  for (int r = 0; r < kSortTile / 256; ++r) {
    const int64_t i = (int64_t)tile * kSortTile + r * 256 + tid;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & 255], 1);
  }
  __syncthreads();
  th[(int64_t)tid * ntiles + tile] = cnt[tid];
}

// exclusive scan of each digit's row th[digit, :] in place (one workgroup of
// 1024 threads per digit), the row's total into dtot[digit]
__global__ __launch_bounds__(1024) void radix_scan_kernel(int* th, int ntiles, int* dtot) {
  __shared__ int part[16];
  const int tid = threadIdx.x;
  int* row = th + (int64_t)blockIdx.x * ntiles;
  const int per = (ntiles + 1023) / 1024, s0 = min(ntiles, tid * per), s1 = min(ntiles, s0 + per);
  int sum = 0;
  for (int i = s0; i < s1; ++i) sum += row[i];
  int total;
  int run = block_scan_1024(sum, part, tid, total);
  for (int i = s0; i < s1; ++i) {
    const int x = row[i];
    row[i] = run;
    run += x;
  }
  if (tid == 0) dtot[blockIdx.x] = total;
}

__global__ __launch_bounds__(256) void radix_scatter_kernel(const uint32_t* __restrict__ kin,
                                                            const int* __restrict__ vin, uint32_t* __restrict__ kout,
                                                            int* __restrict__ vout, int64_t n, int shift,
                                                            const int* __restrict__ th, int ntiles,
                                                            const int* __restrict__ dtot) {
  __shared__ int base[256];
  __shared__ int wcnt[4][256];
  const int tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // digit tid's first output: the counts of all smaller digits plus this
  // digit's count in earlier tiles
  {
    const int t = dtot[tid];
    int x = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wcnt[0][w] = x;
    __syncthreads();
    int pre = x - t;
    for (int k = 0; k < w; ++k) pre += wcnt[0][k];
    base[tid] = pre + th[(int64_t)tid * ntiles + tile];
    __syncthreads();
  }
  const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
  for (int r = 0; r < kSortTile / 256; ++r) {
#pragma unroll
    for (int k = 0; k < 4; ++k) wcnt[k][tid] = 0;
    __syncthreads();
    const int64_t i = (int64_t)tile * kSortTile + r * 256 + tid;
    const bool in = i < n;
    const uint32_t key = in ? kin[i] : 0u;
    const int val = in ? vin[i] : 0;
    const int dg = (int)((key >> shift) & 255);
    uint64_t peers = __ballot(in);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t bb = __ballot((dg >> bit) & 1);
      peers &= ((dg >> bit) & 1) ? bb : ~bb;
    }
    const int below = __popcll(peers & lt);
    if (in && below == 0) wcnt[w][dg] = __popcll(peers);
    __syncthreads();
    if (in) {
      int64_t pos = (int64_t)(unsigned)base[dg] + below;
      for (int k = 0; k < w; ++k) pos += wcnt[k][dg];
      kout[pos] = key;
      vout[pos] = val;
    }
    __syncthreads();
    base[tid] += wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
  }
}

static int sort_key_bits(const Plan& P) {
  int bits = 1;
  while (bits < 32 && ((int64_t)1 << bits) < P.BH * (P.geo.NL + 1)) ++bits;
  return bits;
}

static hipError_t bucket_by_sort(const Plan& P, BucketArgs& a, char* rec, hipStream_t st) {
  const int64_t n = P.B * P.L * P.H * P.S;
  uint32_t* k0 = (uint32_t*)(rec + P.rec.sort_keys);
  uint32_t* k1 = k0 + n;
  int* v0 = (int*)(rec + P.rec.sort_vals);
  int* v1 = v0 + n;
  int* th = (int*)(rec + P.rec.sort_hist);
  const int ntiles = (int)((n + kSortTile - 1) / kSortTile);
  int* dtot = th + (int64_t)256 * ntiles;  // per-digit totals of a pass
  const int64_t ncnt = P.BH * P.geo.NL;
  hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)((ncnt + 255) / 256)), dim3(256), 0, st, a.hist, ncnt);
  hipLaunchKernelGGL(sort_keys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, k0, v0, a.hist, n);
  const int bits = sort_key_bits(P), npass = (bits + 7) / 8;
  for (int ps = 0; ps < npass; ++ps) {
    const int shift = 8 * ps;
    // values ping-pong v0 -> v1 -> v0 ..., the last pass writes `order`
    const uint32_t* kin = ps & 1 ? k1 : k0;
    uint32_t* kout = ps & 1 ? k0 : k1;
    const int* vin = ps & 1 ? v1 : v0;
    int* vout = ps + 1 == npass ? a.order : (ps & 1 ? v0 : v1);
    hipLaunchKernelGGL(radix_hist_kernel, dim3(ntiles), dim3(256), 0, st, kin, n, shift, th, ntiles);
    hipLaunchKernelGGL(radix_scan_kernel, dim3(256), dim3(1024), 0, st, th, ntiles, dtot);
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(ntiles), dim3(256), 0, st, kin, vin, kout, vout, n, shift, th,
                       ntiles, dtot);
  }
  return hipGetLastError();
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
  if (P.bucket_sort) {
    hipError_t e = bucket_by_sort(P, a, rec, st);
    if (e != hipSuccess) return e;
    // nchunk is 1: the scan turns the counts into block starts and pieces
    if (P.nseg > 4) {
      hipLaunchKernelGGL(bucket_segsum_kernel, dim3(P.nseg, P.BH), dim3(1024), 0, st, a);
      hipLaunchKernelGGL(bucket_segscan_kernel, dim3(P.nseg, P.BH), dim3(1024), 0, st, a);
      hipLaunchKernelGGL(bucket_pieces_kernel, dim3(P.BH), dim3(1024), 0, st, a);
    } else {
      hipLaunchKernelGGL(bucket_scan_kernel, dim3(P.BH), dim3(1024), 0, st, a);
    }
    return hipGetLastError();
  }
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
