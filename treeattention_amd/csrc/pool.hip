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
// thread owns 8 contiguous (head, dim) elements and streams the block's rows.
// grid (NL, B); means (B*H, NL, D) float.
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
#pragma unroll 4
    for (int t = 0; t < LB; ++t) {
      float x[8];
      load8f(p + (int64_t)t * sl, x);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += x[i];
    }
    float* o = means + (((int64_t)bb * H + h) * NL + beta) * D + d0;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = acc[i] * inv;
  }
}

struct SumArgs {
  Geo geo;
  int H, D, mode;
  const float* means;   // (BH, NL, D)
  const void* knodes;   // node keys (node-keys mode)
  int64_t ksb, ksl, ksh;
  float* sum32;         // (BH, NS+pad, D)
  void* sum_hi;         // E (BH, NS+pad, D)
  void* sum_lo;         // E
  void* sum_t;          // E or float (BH, D, NS+pad)
};

// One thread per (summary row, dim).  grid (ceil((NS+pad)*D/256), BH).
template <typename E>
__global__ __launch_bounds__(256) void summaries_kernel(SumArgs a) {
  const Geo& G = a.geo;
  const int bh = blockIdx.y;
  const int rows = G.NS;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)rows * a.D) return;
  const int r = (int)(e / a.D), d = (int)(e - (int64_t)r * a.D);
  float val = 0.f;
  int lam = 1;
  while (lam < G.T && r >= G.off[lam + 1]) ++lam;
  const int i = r - G.off[lam];
  if (i < G.pw[lam]) {  // rows past a level's b^lam nodes pad it to a multiple of 32
    if (a.mode == TA_TREE_NATURAL) {
      const int per = G.NL / G.pw[lam];
      const float* m = a.means + ((int64_t)bh * G.NL + (int64_t)i * per) * a.D + d;
      float s = 0.f;
      for (int t = 0; t < per; ++t) s += m[(int64_t)t * a.D];
      val = 0.5f * s / (float)per;
    } else {
      // binary: row = off[d+1] + 2*i' + j for heap node n = 2^d - 1 + i'
      const int depth = lam - 1;
      const int ip = i >> 1, j = i & 1;
      const int n = (1 << depth) - 1 + ip;
      float coef;
      if (a.mode == TA_TREE_COMPAT) {
        const int p = n + 1;
        const int w = p & (-p);
        const float* m = a.means + (int64_t)bh * G.NL * a.D + d;
        float sl = 0.f, sr = 0.f;
        for (int t = 0; t < w; ++t) {
          sl += m[(int64_t)(p - w + t) * a.D];
          sr += m[(int64_t)(p + t) * a.D];
        }
        coef = 0.5f * (sl - sr) / (float)w;
      } else {
        const int bb = bh / a.H, h = bh - bb * a.H;
        const E* kn = (const E*)a.knodes;
        coef = tof(kn[bb * a.ksb + (int64_t)n * a.ksl + h * a.ksh + d]);
      }
      val = j == 0 ? 0.5f * coef : -0.5f * coef;
    }
  }
  const int64_t row_off = ((int64_t)bh * rows + r) * a.D + d;
  a.sum32[row_off] = val;
  const int64_t t_off = ((int64_t)bh * a.D + d) * rows + r;
  if constexpr (sizeof(E) == 2) {
    const E hi = (E)val;
    ((E*)a.sum_hi)[row_off] = hi;
    ((E*)a.sum_lo)[row_off] = (E)(val - (float)hi);
    ((E*)a.sum_t)[t_off] = hi;
  } else {
    ((float*)a.sum_t)[t_off] = val;
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
  a.means = means;
  a.knodes = k;
  a.ksb = P.p.k_strides[0];
  a.ksl = P.p.k_strides[1];
  a.ksh = P.p.k_strides[2];
  a.sum32 = (float*)(rec + P.rec.summaries);
  a.sum_hi = rec + P.rec.sum_hi;
  a.sum_lo = rec + P.rec.sum_lo;
  a.sum_t = rec + P.rec.sum_t;
  const int64_t n = (int64_t)G.NS * P.D;
  hipLaunchKernelGGL(summaries_kernel<E>, dim3((unsigned)((n + 255) / 256), P.BH), dim3(256), 0, st, a);
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
