// K1: per-level key summaries ("pooling").
//
// Natural mode: the child summary of every non-root node is half the mean key
// of its subtree.  Compat mode reproduces the reference's key layout: the
// in-order Haar transform of the leaf-block means (haar_internal_node_keys,
// _treeattn_common.py:54-86, in closed form: coefficient p = (mean of the 2^l
// blocks before p - mean of the 2^l blocks from p) / 2 with l = ctz(p)), read
// in heap order (_tree_mha.py:104,119) and split into the +-k/2 child pair.
// Node-keys mode takes the heap-ordered node keys as given (op-level API).
#include "launch.h"

namespace ta {

__device__ __forceinline__ void load8f(const float* p, float* o) {
  float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void load8f(const bf16* p, float* o) {
  bf16x8 v = *(const bf16x8*)p;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (float)v[i];
}
__device__ __forceinline__ void load8f(const f16* p, float* o) {
  f16x8 v = *(const f16x8*)p;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (float)v[i];
}

// Leaf-block means of the keys: one workgroup per (leaf block, batch), each
// thread owns 8 contiguous (head, dim) elements and streams the block's rows
// with eight 16-byte loads in flight.  grid (NL, B); means (B*H, NL, D) float.
template <typename E>
__global__ __launch_bounds__(256) void block_means_kernel(const E* __restrict__ k, float* __restrict__ means,
                                                          int H, int D, int NL, int LB,
                                                          int64_t sb, int64_t sl, int64_t sh) {
  const int beta = blockIdx.x, bb = blockIdx.y;
  const int nvec = H * D / 8;
  const float inv = 1.f / (float)LB;
  for (int e = threadIdx.x; e < nvec; e += blockDim.x) {
    const int h = (e * 8) / D, d0 = e * 8 - h * D;
    const E* p = k + bb * sb + (int64_t)beta * LB * sl + h * sh + d0;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int t = 0;
    for (; t + 8 <= LB; t += 8) {
      float x[8][8];
#pragma unroll
      for (int j = 0; j < 8; ++j) load8f(p + (int64_t)(t + j) * sl, x[j]);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += x[j][i];
    }
    for (; t < LB; ++t) {
      float x[8];
      load8f(p + (int64_t)t * sl, x);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += x[i];
    }
    float* o = means + (((int64_t)bb * H + h) * NL + beta) * D + d0;
    *(float4*)o = make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
    *(float4*)(o + 4) = make_float4(acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv);
  }
}

// Sums of aligned segments of kSeg block means (and of kSeg such segments),
// so that a summary row over many blocks reads few rows: seg1[j] = sum of
// means j kSeg .. (j + 1) kSeg - 1, seg2[j] = sum of seg1 rows likewise.
// One thread per (segment, 8 dims); grid (ceil(nout D / 8 / 256), BH).
constexpr int kSeg = 64;

__global__ __launch_bounds__(256) void seg_sums_kernel(const float* __restrict__ in, int64_t nin_bh,
                                                       float* __restrict__ out, int64_t nout_bh, int D) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nout_bh * (D / 8)) return;
  const int bh = blockIdx.y;
  const int64_t j = e / (D / 8);
  const int d0 = (int)(e - j * (D / 8)) * 8;
  const float* src = in + ((int64_t)bh * nin_bh + j * kSeg) * D + d0;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int t = 0; t < kSeg; t += 8) {
    float x[8][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) load8f(src + (int64_t)(t + u) * D, x[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += x[u][i];
  }
  float* o = out + ((int64_t)bh * nout_bh + j) * D + d0;
  *(float4*)o = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *(float4*)(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

struct SumArgs {
  Geo geo;
  int H, D, mode;
  int hilo_lam;         // levels 1 .. hilo_lam are read as MFMA tiles: hi copies
  int lo_lam;           // levels 1 .. lo_lam also the lo copies (the sampler's float-accurate tiles)
  int t_lam;            // levels 1 .. t_lam also as the transposed copy
  const float* means;   // (BH, NL, D)
  const float* seg1;    // (BH, NL / kSeg, D) or null
  const float* seg2;    // (BH, NL / kSeg^2, D) or null
  const void* knodes;   // node keys (node-keys mode)
  int64_t ksb, ksl, ksh;
  float* sum32;         // (BH, NS+pad, D)
  void* sum_hi;         // E (BH, NS+pad, D)
  void* sum_lo;         // E
  void* sum_t;          // E or float (BH, D, NS+pad)
};

// acc[0..8) += sum of block means [start, start + count) of this (batch, head)
// (count a power of two, start a multiple of count), from the coarsest
// segment sums that tile the range.
__device__ __forceinline__ void sum_blocks(const SumArgs& a, int bh, int64_t start, int64_t count, int d0,
                                           float* acc) {
  const int D = a.D, NL = a.geo.NL;
  const float* src = a.means + (int64_t)bh * NL * D;
  int64_t n = count, s0 = start;
  if (a.seg2 && count >= kSeg * kSeg) {
    src = a.seg2 + (int64_t)bh * (NL / (kSeg * kSeg)) * D;
    n = count / (kSeg * kSeg);
    s0 = start / (kSeg * kSeg);
  } else if (a.seg1 && count >= kSeg) {
    src = a.seg1 + (int64_t)bh * (NL / kSeg) * D;
    n = count / kSeg;
    s0 = start / kSeg;
  }
  for (int64_t t = 0; t < n; ++t) {
    float x[8];
    load8f(src + (s0 + t) * D + d0, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += x[j];
  }
}

// One workgroup per tile of 32 summary rows of one (batch, head); each
// thread computes 8 dims of one row (vector loads of the block means), writes
// the float, hi and lo rows with 16-byte stores and stages hi in LDS so the
// transposed copy (D, NS) leaves as 32-row (64-byte) pieces per head dim.
// Levels are padded to multiples of 32 rows, so a tile never spans two
// levels.  grid (NS / 32, BH), block 256.
constexpr int kSumRows = 32;

template <typename E>
__global__ __launch_bounds__(256) void summaries_kernel(SumArgs a) {
  const Geo& G = a.geo;
  const int bh = blockIdx.y;
  const int rows = G.NS;
  const int r0 = blockIdx.x * kSumRows;
  const int D = a.D, nv = D / 8;
  __shared__ __align__(16) float tile[kSumRows * (128 + 4)];  // [row][D + 4], hi values as float
  int lam = 1;
  while (lam < G.T && r0 >= G.off[lam + 1]) ++lam;
  for (int e = threadIdx.x; e < kSumRows * nv; e += blockDim.x) {
    const int rr = e / nv, d0 = (e - rr * nv) * 8;
    const int r = r0 + rr;
    const int i = r - G.off[lam];
    float val[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (i < G.pw[lam]) {  // rows past a level's b^lam nodes pad it to a multiple of 32
      if (a.mode == TA_TREE_NATURAL) {
        const int per = G.NL / G.pw[lam];
        sum_blocks(a, bh, (int64_t)i * per, per, d0, val);
        const float f = 0.5f / (float)per;
#pragma unroll
        for (int j = 0; j < 8; ++j) val[j] *= f;
      } else {
        // binary: row = off[d+1] + 2*i' + j for heap node n = 2^d - 1 + i'
        const int depth = lam - 1;
        const int ip = i >> 1, jj = i & 1;
        const int n = (1 << depth) - 1 + ip;
        float coef[8];
        if (a.mode == TA_TREE_COMPAT) {
          const int p = n + 1;
          const int w = p & (-p);
          float sl[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sr[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          sum_blocks(a, bh, p - w, w, d0, sl);
          sum_blocks(a, bh, p, w, d0, sr);
#pragma unroll
          for (int j = 0; j < 8; ++j) coef[j] = 0.5f * (sl[j] - sr[j]) / (float)w;
        } else {
          const int bb = bh / a.H, h = bh - bb * a.H;
          const E* kn = (const E*)a.knodes + bb * a.ksb + (int64_t)n * a.ksl + h * a.ksh + d0;
#pragma unroll
          for (int j = 0; j < 8; ++j) coef[j] = tof(kn[j]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) val[j] = jj == 0 ? 0.5f * coef[j] : -0.5f * coef[j];
      }
    }
    const int64_t row_off = ((int64_t)bh * rows + r) * D + d0;
    *(float4*)(a.sum32 + row_off) = make_float4(val[0], val[1], val[2], val[3]);
    *(float4*)(a.sum32 + row_off + 4) = make_float4(val[4], val[5], val[6], val[7]);
    if (lam > a.hilo_lam) continue;  // per-path levels read the float rows only
    float* tr = tile + rr * (128 + 4) + d0;
    if constexpr (sizeof(E) == 2) {
      typedef __attribute__((ext_vector_type(8))) E e8;
      e8 hi, lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        hi[j] = (E)val[j];
        lo[j] = (E)(val[j] - (float)hi[j]);
        tr[j] = (float)hi[j];
      }
      *(e8*)((E*)a.sum_hi + row_off) = hi;
      if (lam <= a.lo_lam) *(e8*)((E*)a.sum_lo + row_off) = lo;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) tr[j] = val[j];
    }
  }
  if (lam > a.t_lam) return;  // uniform: a tile never spans two levels
  __syncthreads();
  // transposed copy: (bh, d, r0 .. r0 + 31), eight rows per store
  for (int e = threadIdx.x; e < D * (kSumRows / 8); e += blockDim.x) {
    const int d = e / (kSumRows / 8), q0 = (e - d * (kSumRows / 8)) * 8;
    const int64_t t_off = ((int64_t)bh * D + d) * rows + r0 + q0;
    if constexpr (sizeof(E) == 2) {
      typedef __attribute__((ext_vector_type(8))) E e8;
      e8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (E)tile[(q0 + j) * (128 + 4) + d];
      *(e8*)((E*)a.sum_t + t_off) = o;
    } else {
      float* o = (float*)a.sum_t + t_off;
      *(float4*)o = make_float4(tile[q0 * 132 + d], tile[(q0 + 1) * 132 + d], tile[(q0 + 2) * 132 + d],
                                tile[(q0 + 3) * 132 + d]);
      *(float4*)(o + 4) = make_float4(tile[(q0 + 4) * 132 + d], tile[(q0 + 5) * 132 + d],
                                      tile[(q0 + 6) * 132 + d], tile[(q0 + 7) * 132 + d]);
    }
  }
}

__global__ void fill_uniforms_kernel(uint64_t seed, int64_t n, float* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c * 4 >= n) return;
  const Philox4 r = philox4x32_10((uint64_t)c, seed);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (c * 4 + i < n) out[c * 4 + i] = word_to_uniform(r.w[i]);
}

template <typename E>
static hipError_t pool_impl(const Plan& P, const void* k, char* rec, hipStream_t st) {
  const Geo& G = P.geo;
  float* means = (float*)(rec + P.rec.means);
  if (P.p.tree_mode != TA_TREE_NODEKEYS) {
    hipLaunchKernelGGL(block_means_kernel<E>, dim3(G.NL, P.B), dim3(256), 0, st, (const E*)k, means,
                       (int)P.H, (int)P.D, G.NL, G.LB, P.p.k_strides[0], P.p.k_strides[1],
                       P.p.k_strides[2]);
  }
  SumArgs a;
  a.geo = G;
  a.H = (int)P.H;
  a.D = (int)P.D;
  a.mode = P.p.tree_mode;
  // level lam holds the children of depth lam - 1 nodes: MFMA tiles in the
  // sampler below depth sample_dense (and, causal, the boundary nodes' children
  // at every depth), in the tree backward below tree_dense (also transposed),
  // or with path rows every level's path children in the leaf backward (not
  // transposed)
  a.t_lam = P.path_rows || P.leaf_path ? 0 : P.tree_dense;
  a.hilo_lam = P.p.causal == TA_CAUSAL_EXACT || P.path_rows || P.leaf_path
                   ? G.T
                   : (P.sample_dense > P.tree_dense ? P.sample_dense : P.tree_dense);
  a.lo_lam = P.p.causal == TA_CAUSAL_EXACT ? G.T : P.sample_dense;  // the backward reads hi only
  a.means = means;
  a.knodes = k;
  a.ksb = P.p.k_strides[0];
  a.ksl = P.p.k_strides[1];
  a.ksh = P.p.k_strides[2];
  a.sum32 = (float*)(rec + P.rec.summaries);
  a.sum_hi = rec + P.rec.sum_hi;
  a.sum_lo = rec + P.rec.sum_lo;
  a.sum_t = rec + P.rec.sum_t;
  a.seg1 = a.seg2 = nullptr;
  if (P.p.tree_mode != TA_TREE_NODEKEYS && G.NL >= 2 * kSeg) {
    float* s1 = (float*)(rec + P.rec.segs);
    const int64_t n1 = G.NL / kSeg, n2 = G.NL / (kSeg * kSeg);
    hipLaunchKernelGGL(seg_sums_kernel, dim3((unsigned)((n1 * (P.D / 8) + 255) / 256), P.BH), dim3(256), 0, st,
                       (const float*)means, (int64_t)G.NL, s1, n1, (int)P.D);
    a.seg1 = s1;
    if (n2 >= 2) {
      float* s2 = s1 + P.BH * n1 * P.D;
      hipLaunchKernelGGL(seg_sums_kernel, dim3((unsigned)((n2 * (P.D / 8) + 255) / 256), P.BH), dim3(256), 0, st,
                         (const float*)s1, n1, s2, n2, (int)P.D);
      a.seg2 = s2;
    }
  }
  if (G.NS > 0)
    hipLaunchKernelGGL(summaries_kernel<E>, dim3((unsigned)(G.NS / kSumRows), P.BH), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_pool(const Plan& P, const void* k, char* rec, hipStream_t st) {
  switch (P.p.dtype) {
    case TA_F32: return pool_impl<float>(P, k, rec, st);
    case TA_BF16: return pool_impl<bf16>(P, k, rec, st);
    default: return pool_impl<f16>(P, k, rec, st);
  }
}

hipError_t launch_fill_uniforms(uint64_t seed, int64_t n, float* out, hipStream_t st) {
  const int64_t nc = (n + 3) / 4;
  if (nc == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_uniforms_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, seed, n, out);
  return hipGetLastError();
}

}  // namespace ta
