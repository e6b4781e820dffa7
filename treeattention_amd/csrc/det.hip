// Deterministic (exact) tree attention on the reference tree: binary, one
// token per leaf, heap-ordered node keys (_tree_mha.py:271-321).
//
// Query l reaches leaf n with probability prod_d sigma(+-x), x = q_l . k_node
// over the n's root-to-leaf path (left child: sigma(x), right: sigma(-x),
// _tree_mha.py:287-306).  Non-causal weights are those probabilities; causal
// weights are their softmax over the leaves n <= l (:308-314).  The dense
// products (node logits X = Q K^T, out = W V and the gradient products) are
// plain batched GEMMs; these kernels do the tree-structured parts per row
// (one (batch, head, query) row per workgroup):
//   det_weights_kernel: X row -> leaf log-probabilities by a top-down level
//     recursion (lp[2i + c] = lp[i] + logsig(+-x), logsig(-x) = logsig(x) - x),
//     then exp or the causal softmax;
//   det_grad_kernel:    W, dW rows -> dlogw = W (dW - delta) (delta = sum W dW
//     when causal, 0 otherwise), bottom-up subtree sums A, and the node-logit
//     gradient G = sigma(-x) A_left - sigma(x) A_right, written over X;
//   haar_keys_kernel / haar_keys_adjoint_kernel: the heap-ordered Haar node
//     keys of the attn-bench adapter (_treeattn_common.py:54-86) and the
//     transpose of that linear map.
#include "launch.h"

namespace ta {

// One workgroup of kDetThreads per row.  The top kDetTop levels of the tree
// (2^kDetTop subtree roots) run level by level through LDS; below them thread
// t owns the subtree of root t, C = N >> kDetTop leaves, processed in chunks
// of up to 16 leaves whose last four levels are a register recursion (no
// barriers): the forward walks root -> chunk root -> leaves, the backward
// leaves -> chunk root -> subtree root -> top levels.
constexpr int kDetThreads = 256;
constexpr int kDetTop = 8;  // 2^kDetTop == kDetThreads
constexpr int kDetChunks = kDetMaxLeaves / kDetThreads / 16;  // chunks per thread at most

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
  return s;
}
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = -__builtin_inff();
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s = fmaxf(s, red[i]);
  return s;
}

// Heap index of the node at depth dd on the path to leaf n of a depth-T tree.
__device__ __forceinline__ int path_node(int dd, int n, int T) { return (1 << dd) - 1 + (n >> (T - dd)); }

// grid: rows (B*H*L), block kDetThreads, dynamic LDS N floats when causal.
__global__ __launch_bounds__(kDetThreads) void det_weights_kernel(const float* __restrict__ X, int64_t ldx,
                                                                  float* __restrict__ W, int64_t ldw, int L, int N,
                                                                  int T, int causal) {
  extern __shared__ float lp[];  // causal: the row's leaf log-probabilities
  __shared__ float top[2][kDetThreads];
  __shared__ float red[kDetThreads / 64];
  const int64_t r = blockIdx.x;
  const int l = (int)(r % L);
  const int tid = threadIdx.x;
  const float* x = X + r * ldx;
  float* w = W + r * ldw;
  const int tb = min(T, kDetTop), c = T - tb, C = 1 << c;
  const int cl = min(c, 4), nchunk = C >> cl;
  const bool vec = (reinterpret_cast<uintptr_t>(w) & 15) == 0;  // 16-byte row stores

  int cur = 0;
  if (tid == 0) top[0][0] = 0.f;
  __syncthreads();
  for (int d = 0; d < tb; ++d) {
    const int nd = 1 << d;
    if (tid < nd) {
      const float a = top[cur][tid], xv = x[nd - 1 + tid];
      const float ls = logsig(xv);
      top[cur ^ 1][2 * tid] = a + ls;
      top[cur ^ 1][2 * tid + 1] = a + ls - xv;
    }
    cur ^= 1;
    __syncthreads();
  }
  float mx = -__builtin_inff();
  if (tid < (1 << tb)) {
    const float root = top[cur][tid];
    for (int j = 0; j < nchunk; ++j) {
      const int base = tid * C + (j << cl);
      float p = root;
      for (int dd = tb; dd < T - cl; ++dd) {  // subtree root -> chunk root
        const float xv = x[path_node(dd, base, T)];
        const float ls = logsig(xv);
        p += ((base >> (T - 1 - dd)) & 1) ? ls - xv : ls;
      }
      float a[16];
      a[0] = p;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e < cl) {
          const int n0 = path_node(T - cl + e, base, T);
#pragma unroll
          for (int i = (1 << e) - 1; i >= 0; --i) {  // descending: a[2i], a[2i+1] overwrite nothing unread
            const float xv = x[n0 + i];
            const float ls = logsig(xv);
            a[2 * i + 1] = a[i] + ls - xv;
            a[2 * i] = a[i] + ls;
          }
        }
      }
      const int m = 1 << cl;
      if (causal) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < m) {
            lp[base + i] = a[i];
            if (base + i <= l) mx = fmaxf(mx, a[i]);
          }
      } else if (m == 16 && vec) {
#pragma unroll
        for (int i = 0; i < 16; i += 4)
          *(float4*)(w + base + i) = make_float4(expf(a[i]), expf(a[i + 1]), expf(a[i + 2]), expf(a[i + 3]));
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < m) w[base + i] = expf(a[i]);
      }
    }
  }
  if (causal) {
    mx = block_max(mx, red);  // includes a barrier: lp is complete
    float s = 0.f;
    for (int n = tid; n <= l && n < N; n += kDetThreads) s += expf(lp[n] - mx);
    s = block_sum(s, red);
    const float inv = 1.f / s;
    for (int n = tid; n < N; n += kDetThreads) w[n] = n <= l ? expf(lp[n] - mx) * inv : 0.f;
  }
}

// grid: rows, block kDetThreads.  G overwrites X.
__global__ __launch_bounds__(kDetThreads) void det_grad_kernel(float* __restrict__ XG, int64_t ldx,
                                                               const float* __restrict__ W, const float* __restrict__ dW,
                                                               int64_t ldw, int N, int T, int causal) {
  __shared__ float top[2][kDetThreads];
  __shared__ float red[kDetThreads / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const float* w = W + r * ldw;
  const float* dw = dW + r * ldw;
  float* xg = XG + r * ldx;
  const int tb = min(T, kDetTop), c = T - tb, C = 1 << c;
  const int cl = min(c, 4), nchunk = C >> cl;
  float delta = 0.f;
  if (causal) {
    float s = 0.f;
    for (int n = tid; n < N; n += kDetThreads) s += w[n] * dw[n];
    delta = block_sum(s, red);
  }
  // node gradient from the two children's summed dlogw; returns the parent's sum
  auto node = [&](int nidx, float al, float ar) {
    const float xv = xg[nidx];
    const float sg = 1.f / (1.f + expf(-xv));
    xg[nidx] = (1.f - sg) * al - sg * ar;
    return al + ar;
  };
  float total = 0.f;
  if (tid < (1 << tb)) {
    float ct[kDetChunks];
#pragma unroll
    for (int j = 0; j < kDetChunks; ++j) {
      if (j < nchunk) {
        const int base = tid * C + (j << cl);
        const int m = 1 << cl;
        float a[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < m) a[i] = w[base + i] * (dw[base + i] - delta);
#pragma unroll
        for (int e = 3; e >= 0; --e) {
          if (e < cl) {
            const int n0 = path_node(T - cl + e, base, T);
#pragma unroll
            for (int i = 0; i < (1 << e); ++i) a[i] = node(n0 + i, a[2 * i], a[2 * i + 1]);
          }
        }
        ct[j] = a[0];
      }
    }
    // chunk roots (depth T - cl) -> subtree root (depth tb): at most three levels
#pragma unroll
    for (int e = 2; e >= 0; --e) {
      if (e < c - cl) {
        const int n0 = path_node(tb + e, tid * C, T);
#pragma unroll
        for (int i = 0; i < (1 << e); ++i) ct[i] = node(n0 + i, ct[2 * i], ct[2 * i + 1]);
      }
    }
    total = ct[0];
  }
  int cur = 0;
  top[0][tid] = total;
  __syncthreads();
  for (int d = tb - 1; d >= 0; --d) {
    const int nd = 1 << d;
    if (tid < nd) top[cur ^ 1][tid] = node(nd - 1 + tid, top[cur][2 * tid], top[cur][2 * tid + 1]);
    cur ^= 1;
    __syncthreads();
  }
}

// Heap node m of an N-leaf binary tree (p = m + 1, w = lowest set bit of p):
// key = (mean of k[p-w, p) - mean of k[p, p+w)) / 2, the in-order Haar
// coefficient p of the keys read in heap order (_treeattn_common.py:70-86,
// _tree_mha.py:104,119).  Output (K, B, H, D) float; one thread per
// (m, b, h, 4 dims).
template <typename E>
__global__ __launch_bounds__(256) void haar_keys_kernel(const E* __restrict__ k, int64_t sb, int64_t sl, int64_t sh,
                                                        float* __restrict__ out, int B, int H, int D, int N) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int D4 = D / 4;
  const int64_t total = (int64_t)(N - 1) * B * H * D4;
  if (e >= total) return;
  const int d0 = (int)(e % D4) * 4;
  const int64_t mbh = e / D4;
  const int h = (int)(mbh % H);
  const int64_t mb = mbh / H;
  const int bb = (int)(mb % B);
  const int m = (int)(mb / B);
  const int p = m + 1, w = p & (-p);
  const E* base = k + bb * sb + h * sh + d0;
  float sl_[4] = {0, 0, 0, 0}, sr_[4] = {0, 0, 0, 0};
  for (int t = 0; t < w; ++t) {
    const E* a = base + (int64_t)(p - w + t) * sl;
    const E* c = base + (int64_t)(p + t) * sl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sl_[i] += tof(a[i]);
      sr_[i] += tof(c[i]);
    }
  }
  const float f = 0.5f / (float)w;
  float* o = out + (((int64_t)m * B + bb) * H + h) * D + d0;
  *(float4*)o = make_float4((sl_[0] - sr_[0]) * f, (sl_[1] - sr_[1]) * f, (sl_[2] - sr_[2]) * f,
                            (sl_[3] - sr_[3]) * f);
}

// The same keys from a block-sum pyramid, O(N D) work per (batch, head): at
// level l (w = 2^l) the nodes are p = (2j + 1) w, with key (BS_l[2j] -
// BS_l[2j+1]) / 2w for the block sums BS_l of w keys, and BS_{l+1}[j] =
// BS_l[2j] + BS_l[2j+1].  haar_seg_kernel runs the levels inside segments of
// kHaarSeg tokens in LDS (one workgroup per segment and (batch, head)) and
// leaves each segment's sum; haar_top_kernel runs the levels above on the
// segment sums (one workgroup per (batch, head) and 16 head dims).
constexpr int kHaarSeg = 128;
constexpr int kHaarTopDims = 16;

template <typename E>
__global__ __launch_bounds__(256) void haar_seg_kernel(const E* __restrict__ k, int64_t sb, int64_t sl, int64_t sh,
                                                       float* __restrict__ out, float* __restrict__ segsum, int B,
                                                       int H, int D, int seg) {
  extern __shared__ __align__(16) float buf[];  // [seg][D]
  const int s = blockIdx.x, bh = blockIdx.y, bb = bh / H, h = bh - bb * H;
  const int t0 = s * seg, D4 = D / 4;
  for (int e = threadIdx.x; e < seg * D4; e += 256) {
    const int tok = e / D4, d0 = (e - tok * D4) * 4;
    const E* src = k + bb * sb + (int64_t)(t0 + tok) * sl + h * sh + d0;
    *(float4*)(buf + tok * D + d0) = make_float4(tof(src[0]), tof(src[1]), tof(src[2]), tof(src[3]));
  }
  __syncthreads();
  for (int lv = 0; (2 << lv) <= seg; ++lv) {
    const int w = 1 << lv, npair = seg >> (lv + 1);
    const float f = 0.5f / (float)w;
    for (int e = threadIdx.x; e < npair * D4; e += 256) {
      const int j = e / D4, d0 = (e - j * D4) * 4;
      float* pa = buf + (2 * j * w) * D + d0;
      const float4 a = *(const float4*)pa, b = *(const float4*)(pa + w * D);
      const int64_t m = (int64_t)t0 + (2 * j + 1) * w - 1;
      *(float4*)(out + ((m * B + bb) * H + h) * D + d0) =
          make_float4((a.x - b.x) * f, (a.y - b.y) * f, (a.z - b.z) * f, (a.w - b.w) * f);
      *(float4*)pa = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    }
    __syncthreads();
  }
  if (segsum)
    for (int e = threadIdx.x; e < D4; e += 256)
      *(float4*)(segsum + ((int64_t)bh * gridDim.x + s) * D + 4 * e) = *(const float4*)(buf + 4 * e);
}

__global__ __launch_bounds__(256) void haar_top_kernel(const float* __restrict__ segsum, float* __restrict__ out,
                                                       int B, int H, int D, int nseg, int seg) {
  extern __shared__ __align__(16) float tb[];  // [nseg][kHaarTopDims]
  const int bh = blockIdx.x, bb = bh / H, h = bh - bb * H, dc = blockIdx.y * kHaarTopDims;
  for (int e = threadIdx.x; e < nseg * kHaarTopDims; e += 256) {
    const int sg = e / kHaarTopDims, d = e - sg * kHaarTopDims;
    tb[e] = dc + d < D ? segsum[((int64_t)bh * nseg + sg) * D + dc + d] : 0.f;
  }
  __syncthreads();
  for (int lv = 0; (2 << lv) <= nseg; ++lv) {
    const int ws = 1 << lv, npair = nseg >> (lv + 1);
    const int64_t wt = (int64_t)ws * seg;  // block width in tokens
    const float f = 0.5f / (float)wt;
    for (int e = threadIdx.x; e < npair * kHaarTopDims; e += 256) {
      const int j = e / kHaarTopDims, d = e - j * kHaarTopDims;
      float* pa = tb + (2 * j * ws) * kHaarTopDims + d;
      const float a = pa[0], b = pa[ws * kHaarTopDims];
      const int64_t m = (2 * j + 1) * wt - 1;
      if (dc + d < D) out[((m * B + bb) * H + h) * D + dc + d] = (a - b) * f;
      pa[0] = a + b;
    }
    __syncthreads();
  }
}

// dk[b, t, h, :] = sum over the levels l of +-dkey[m_l] / 2^(l+1): at level l
// leaf t lies in the left (+) or right (-) span of exactly one coefficient,
// p_l = (t >> (l+1) << (l+1)) + 2^l.  One thread per (t, b, h, 4 dims).
template <typename E>
__global__ __launch_bounds__(256) void haar_keys_adjoint_kernel(const float* __restrict__ dkey, E* __restrict__ dk,
                                                                int64_t sb, int64_t sl, int64_t sh, int B, int H, int D,
                                                                int N, int T) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int D4 = D / 4;
  const int64_t total = (int64_t)N * B * H * D4;
  if (e >= total) return;
  const int d0 = (int)(e % D4) * 4;
  const int64_t tbh = e / D4;
  const int h = (int)(tbh % H);
  const int64_t tb = tbh / H;
  const int bb = (int)(tb % B);
  const int t = (int)(tb / B);
  float acc[4] = {0, 0, 0, 0};
  for (int l = 0; l < T; ++l) {
    const int p = ((t >> (l + 1)) << (l + 1)) + (1 << l);
    const float f = (((t >> l) & 1) ? -0.5f : 0.5f) / (float)(1 << l);
    const float4 g = *(const float4*)(dkey + (((int64_t)(p - 1) * B + bb) * H + h) * D + d0);
    acc[0] += f * g.x;
    acc[1] += f * g.y;
    acc[2] += f * g.z;
    acc[3] += f * g.w;
  }
  E* o = dk + bb * sb + (int64_t)t * sl + h * sh + d0;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (E)acc[i];
}

hipError_t launch_det_weights(const float* X, int64_t ldx, float* W, int64_t ldw, int64_t rows, int L, int N, int T,
                              int causal, hipStream_t st) {
  const int smem = causal ? N * 4 : 0;
  hipError_t e = hipFuncSetAttribute((const void*)det_weights_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(det_weights_kernel, dim3((unsigned)rows), dim3(kDetThreads), smem, st, X, ldx, W, ldw, L, N, T,
                     causal);
  return hipGetLastError();
}

hipError_t launch_det_grad(float* XG, int64_t ldx, const float* W, const float* dW, int64_t ldw, int64_t rows, int N,
                           int T, int causal, hipStream_t st) {
  hipLaunchKernelGGL(det_grad_kernel, dim3((unsigned)rows), dim3(kDetThreads), 0, st, XG, ldx, W, dW, ldw, N, T,
                     causal);
  return hipGetLastError();
}

template <typename E>
static hipError_t haar_keys_t(const void* k, const int64_t* ks, float* out, float* segsum, int B, int H, int D,
                              int N, hipStream_t st) {
  const int64_t total = (int64_t)(N - 1) * B * H * (D / 4);
  if (total == 0) return hipSuccess;
  const int seg = N < kHaarSeg ? N : kHaarSeg, nseg = N / seg;
  const int smem = seg * D * 4;
  if (segsum && smem <= 160 * 1024 && nseg * kHaarTopDims * 4 <= 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)haar_seg_kernel<E>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(haar_seg_kernel<E>, dim3((unsigned)nseg, (unsigned)(B * H)), dim3(256), smem, st,
                       (const E*)k, ks[0], ks[1], ks[2], out, nseg > 1 ? segsum : nullptr, B, H, D, seg);
    e = hipGetLastError();
    if (e != hipSuccess || nseg == 1) return e;
    hipLaunchKernelGGL(haar_top_kernel, dim3((unsigned)(B * H), (unsigned)((D + kHaarTopDims - 1) / kHaarTopDims)),
                       dim3(256), nseg * kHaarTopDims * 4, st, segsum, out, B, H, D, nseg, seg);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(haar_keys_kernel<E>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, (const E*)k, ks[0],
                     ks[1], ks[2], out, B, H, D, N);
  return hipGetLastError();
}

hipError_t launch_haar_keys(int dtype, const void* k, const int64_t* ks, float* out, float* segsum, int B, int H,
                            int D, int N, hipStream_t st) {
  switch (dtype) {
    case TA_F32: return haar_keys_t<float>(k, ks, out, segsum, B, H, D, N, st);
    case TA_BF16: return haar_keys_t<bf16>(k, ks, out, segsum, B, H, D, N, st);
    default: return haar_keys_t<f16>(k, ks, out, segsum, B, H, D, N, st);
  }
}

int64_t haar_workspace_floats(int B, int H, int D, int N) {
  const int seg = N < kHaarSeg ? N : kHaarSeg;
  return (int64_t)B * H * (N / seg) * D;
}

template <typename E>
static hipError_t haar_adj_t(const float* dkey, void* dk, const int64_t* ks, int B, int H, int D, int N, int T,
                             hipStream_t st) {
  const int64_t total = (int64_t)N * B * H * (D / 4);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(haar_keys_adjoint_kernel<E>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, dkey,
                     (E*)dk, ks[0], ks[1], ks[2], B, H, D, N, T);
  return hipGetLastError();
}

hipError_t launch_haar_keys_adjoint(int dtype, const float* dkey, void* dk, const int64_t* ks, int B, int H, int D,
                                    int N, int T, hipStream_t st) {
  switch (dtype) {
    case TA_F32: return haar_adj_t<float>(dkey, dk, ks, B, H, D, N, T, st);
    case TA_BF16: return haar_adj_t<bf16>(dkey, dk, ks, B, H, D, N, T, st);
    default: return haar_adj_t<f16>(dkey, dk, ks, B, H, D, N, T, st);
  }
}

}  // namespace ta
